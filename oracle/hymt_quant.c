/*
 * hymt_quant.c -- CPU restatement of the reference's quantized weight rows.
 *
 * TEST INFRASTRUCTURE ONLY (see hymt_oracle.h): the parity checker for the
 * HIP weight GEMVs in hymt2sharp_amd/csrc/gemv.hip.
 *
 * orc_dequant_row restates the DequantizeRow of each block format the
 * reference's models use (src/HyMT2Sharp/Kernels), on the GGUF block bytes
 * exactly as GgufFile hands them to the kernels:
 *   Q8_0    Q8_0.cs:16-35        32 values: fp16 d, int8 q; y = d q
 *   Q4_K    Q4K.cs:8-19, 36-61   256 values: fp16 d, dmin, 12 bytes of 6-bit
 *                                scales/mins (GetScaleMin), 128 nibble bytes
 *   Q6_K    Q6K.cs:37-66         256 values: ql[128], qh[64], int8 scales[16],
 *                                fp16 d; q = 6-bit - 32
 *   Q2_0C   Q2_0C.cs:13-26       512 values: fp16 d, 128 bytes of 2-bit codes,
 *                                value (2c - 3) d
 *   STQ1_0  STQ1_0.cs:57-101     256 values: 64 groups, 4-bit codebook slot +
 *                                1 sign bit per group, fp16 d; a group holds
 *                                four ternary lanes strided by 16
 * and F32 / F16 rows.  Block structs: BlockLayout.cs:9-106; fp16 scales:
 * HalfBits.ToSingle (BlockLayout.cs:216-245), exact like orc_f16_to_f32.
 *
 * orc_gemv is y = W x over the dequantized rows, accumulated in double: the
 * exact product of the stored weights and the fp32 activations, which the
 * GPU kernels are held to within fp32 summation error.  (The reference CPU
 * path quantizes activations to Q8_K first, KQuantGemv.cs; that is a
 * different rounding, not a property of the weights.)
 */
#include <stdint.h>
#include <string.h>

#include "hymt_oracle.h"

#define T_F32 0
#define T_F16 1
#define T_Q8_0 8
#define T_Q4_K 12
#define T_Q6_K 14
#define T_Q2_0C 40
#define T_STQ1_0 43

static float h2f(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* Q4K.GetScaleMin (Q4K.cs:8-19) */
static void scale_min_k4(int j, const uint8_t *s, int *sc, int *m)
{
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* STQ1_0.Codebook (STQ1_0.cs:57-63): four 2-bit lanes, 0 = -1, 1 = 0, 2 = +1 */
static const uint8_t stq_codebook[32] = {
    0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42,
    0x01, 0x21, 0x81, 0xA1, 0x04, 0x24, 0x84, 0xA4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68,
};

long orc_row_bytes(int type, int n)
{
    switch (type) {
    case T_F32: return 4L * n;
    case T_F16: return 2L * n;
    case T_Q8_0: return n / 32 * 34L;
    case T_Q4_K: return n / 256 * 144L;
    case T_Q6_K: return n / 256 * 210L;
    case T_Q2_0C: return n / 512 * 130L;
    case T_STQ1_0: return n / 256 * 42L;
    default: return -1;
    }
}

int orc_dequant_row(int type, const void *row, int n, float *y)
{
    const uint8_t *p = (const uint8_t *)row;
    switch (type) {
    case T_F32:
        memcpy(y, p, 4L * n);
        return 0;
    case T_F16:
        for (int i = 0; i < n; i++) y[i] = h2f(p + 2 * i);
        return 0;
    case T_Q8_0: /* Q8_0.cs:16-35 */
        for (int b = 0; b < n / 32; b++, p += 34) {
            const float d = h2f(p);
            for (int j = 0; j < 32; j++) y[b * 32 + j] = d * (float)(int8_t)p[2 + j];
        }
        return 0;
    case T_Q4_K: /* Q4K.cs:36-61 */
        for (int b = 0; b < n / 256; b++, p += 144) {
            const float d = h2f(p), dmin = h2f(p + 2);
            const uint8_t *sc = p + 4, *q = p + 16;
            float *o = y + 256 * b;
            for (int j = 0, is = 0; j < 256; j += 64, is += 2, q += 32) {
                int s0, m0, s1, m1;
                scale_min_k4(is, sc, &s0, &m0);
                scale_min_k4(is + 1, sc, &s1, &m1);
                const float d1 = d * s0, mm1 = dmin * m0, d2 = d * s1, mm2 = dmin * m1;
                for (int l = 0; l < 32; l++) *o++ = d1 * (q[l] & 0xF) - mm1;
                for (int l = 0; l < 32; l++) *o++ = d2 * (q[l] >> 4) - mm2;
            }
        }
        return 0;
    case T_Q6_K: /* Q6K.cs:37-66 */
        for (int b = 0; b < n / 256; b++, p += 210) {
            const uint8_t *ql = p, *qh = p + 128;
            const int8_t *sc = (const int8_t *)(p + 192);
            const float d = h2f(p + 208);
            float *o = y + 256 * b;
            for (int h = 0; h < 2; h++, ql += 64, qh += 32, sc += 8, o += 128)
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const int q1 = (ql[l] & 0xF) | ((qh[l] & 3) << 4);
                    const int q2 = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
                    const int q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
                    const int q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
                    o[l] = d * sc[is] * (q1 - 32);
                    o[l + 32] = d * sc[is + 2] * (q2 - 32);
                    o[l + 64] = d * sc[is + 4] * (q3 - 32);
                    o[l + 96] = d * sc[is + 6] * (q4 - 32);
                }
        }
        return 0;
    case T_Q2_0C: /* Q2_0C.cs:13-26: Value = ((b >> shift) & 3) * 2 - 3 */
        for (int b = 0; b < n / 512; b++, p += 130) {
            const float d = h2f(p);
            for (int j = 0; j < 512; j++) y[b * 512 + j] = (float)((((p[2 + j / 4] >> ((j & 3) * 2)) & 3) * 2) - 3) * d;
        }
        return 0;
    case T_STQ1_0: /* STQ1_0.cs:66-101 */
        for (int b = 0; b < n / 256; b++, p += 42) {
            const uint8_t *qs = p, *sign = p + 32;
            const float d = h2f(p + 40);
            for (int g = 0; g < 64; g++) {
                const int slot = (qs[g >> 1] >> ((g & 1) * 4)) & 0x0F;
                const int sg = (sign[g >> 3] >> (g & 7)) & 1;
                const int qpack = stq_codebook[(sg << 4) | slot];
                const int chunk = g >> 4, gloc = g & 15;
                for (int lane = 0; lane < 4; lane++)
                    y[b * 256 + chunk * 64 + gloc + lane * 16] = (float)(((qpack >> (lane * 2)) & 3) - 1) * d;
            }
        }
        return 0;
    default:
        return -1;
    }
}

/* y[r] (+)= sum_c W[r][c] x[c] over the dequantized rows, in double */
int orc_gemv(int type, const void *w, int rows, int cols, const float *x, float *y, int accumulate)
{
    const long rb = orc_row_bytes(type, cols);
    if (rb < 0) return -1;
    float row[32768];
    if (cols > 32768) return -2;
    for (int r = 0; r < rows; r++) {
        if (orc_dequant_row(type, (const uint8_t *)w + rb * r, cols, row)) return -1;
        double s = 0;
        for (int c = 0; c < cols; c++) s += (double)row[c] * (double)x[c];
        y[r] = accumulate ? (float)((double)y[r] + s) : (float)s;
    }
    return 0;
}
