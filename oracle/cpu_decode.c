/*
 * cpu_decode.c -- C restatement of the reference's CPU decode step, the
 * path its published CPU figures come from (README_EN.md:132,138): every
 * projection quantizes its fp32 input to Q8_K once and runs integer dots
 * against the Q4_K / Q6_K weight blocks.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it and
 * tests/test_cpu_decode_port.py pins it; the product never links it.
 *
 *   q8k_quantize      Q8K.QuantizeRow + ScaleBlock (Kernels/Q8K.cs:12-137):
 *                     d = 1 / (-127 / max), max the first signed extremum of
 *                     the 256-value block, q = clamp(rne(x * iscale), +-127),
 *                     bsums over runs of 16
 *   dot_q4k           VecDotQ4K.Dot (Kernels/VecDotQ4K.cs:11-20): per block
 *                     d_y d_x sum_j sc_j (q4 . q8)_j - d_y dmin_x sum_j mn_j bsum_j
 *   dot_q6k           Q6K.Dot (Kernels/Q6K.cs): d_y d_x sum_g sc_g (q6 - 32) . q8
 *   rows over threads KQuantGemv.Multi (Kernels/KQuantGemv.cs:19-72): the q, k
 *                     and v (or gate and up) rows share one quantized input,
 *                     dynamic chunks of max(8, rows / (16 threads)) rows
 *   the step          HunyuanDenseModel.Decode.cs:30-101 (DecodeBlock,
 *                     DecodeAttention, DecodeQkv, DecodeGateUp, DecodeLinear):
 *                     RMSNorm, q/k/v, RoPE + QK norm + bf16 append + attention
 *                     (orc_decode_attention), o projection, residual, RMSNorm,
 *                     gate/up, SiLU * up, down, residual; then the output norm
 *                     and projection (HunyuanDenseModel.cs:390-419)
 *
 * The integer dots are written with AVX2 (unsigned x signed byte products
 * summed in 16-bit pairs, then weighted by the block scales in 32-bit), the
 * same instruction tier as the reference's DotAvx2 kernels; the sums are
 * exact integers, so the order does not change them.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "hymt_oracle.h"

#define T_Q4_K 12
#define T_Q6_K 14

typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} q8k_block;

static float h2f(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* Q8K.QuantizeRow / ScaleBlock (Q8K.cs:12-137) */
static void q8k_quantize(const float *x, q8k_block *y, int n)
{
    for (int b = 0; b < n / 256; b++) {
        const float *src = x + 256 * b;
        float amax = 0.0f;
        for (int j = 0; j < 256; j++) amax = fmaxf(amax, fabsf(src[j]));
        if (amax == 0.0f) {
            memset(&y[b], 0, sizeof(q8k_block));
            continue;
        }
        float max = 0.0f;
        for (int j = 0; j < 256; j++)
            if (fabsf(src[j]) == amax) {
                max = src[j];
                break;
            }
        const float iscale = -127.0f / max;
        y[b].d = 1.0f / iscale;
        for (int j = 0; j < 256; j++) {
            float r = nearbyintf(src[j] * iscale);
            r = r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
            y[b].qs[j] = (int8_t)r;
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int j = 0; j < 16; j++) s += y[b].qs[16 * g + j];
            y[b].bsums[g] = (int16_t)s;
        }
    }
}

static int hsum8(__m256i v)
{
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

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

/* VecDotQ4K.Dot: 144-byte blocks (d, dmin, 12 scale bytes, 128 nibble bytes) */
static float dot_q4k(const uint8_t *w, const q8k_block *y, int nb)
{
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    float sum = 0.0f;
    for (int b = 0; b < nb; b++, w += 144, y++) {
        const float d = y->d * h2f(w), dmin = y->d * h2f(w + 2);
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) scale_min_k4(j, w + 4, &sc[j], &mn[j]);
        int summs = 0;
        for (int j = 0; j < 8; j++) summs += mn[j] * (y->bsums[2 * j] + y->bsums[2 * j + 1]);
        const uint8_t *q = w + 16;
        __m256i acc = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            const __m256i q4 = _mm256_loadu_si256((const __m256i *)(q + 32 * j));
            const __m256i lo = _mm256_and_si256(q4, m4), hi = _mm256_and_si256(_mm256_srli_epi16(q4, 4), m4);
            const __m256i a0 = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * j));
            const __m256i a1 = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * j + 32));
            const __m256i p0 = _mm256_maddubs_epi16(lo, a0), p1 = _mm256_maddubs_epi16(hi, a1);
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p0, _mm256_set1_epi16((short)sc[2 * j])));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p1, _mm256_set1_epi16((short)sc[2 * j + 1])));
        }
        sum += d * (float)hsum8(acc) - dmin * (float)summs;
    }
    return sum;
}

/* Q6K.Dot: 210-byte blocks (128 low-nibble bytes, 64 high-bit bytes, 16 int8
 * scales, fp16 d); value = (nibble | 2 high bits << 4) - 32 */
static float dot_q6k(const uint8_t *w, const q8k_block *y, int nb)
{
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(0x03);
    float sum = 0.0f;
    for (int b = 0; b < nb; b++, w += 210, y++) {
        const int8_t *sc = (const int8_t *)(w + 192);
        const float d = y->d * h2f(w + 208);
        int off = 0;
        for (int g = 0; g < 16; g++) off += sc[g] * y->bsums[g];
        __m256i acc = _mm256_setzero_si256();
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = w + 64 * h, *qh = w + 128 + 32 * h;
            const __m256i l0 = _mm256_loadu_si256((const __m256i *)ql);
            const __m256i l1 = _mm256_loadu_si256((const __m256i *)(ql + 32));
            const __m256i hb = _mm256_loadu_si256((const __m256i *)qh);
            __m256i qv[4];
            qv[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(hb, m2), 4));
            qv[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 2), m2), 4));
            qv[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 4), m2), 4));
            qv[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 6), m2), 4));
            for (int k = 0; k < 4; k++) {
                /* values 128 h + 32 k + [0, 32): scale groups 8 h + 2 k and 8 h + 2 k + 1 */
                const __m256i a = _mm256_loadu_si256((const __m256i *)(y->qs + 128 * h + 32 * k));
                const __m256i p = _mm256_maddubs_epi16(qv[k], a);
                const short s0 = sc[8 * h + 2 * k], s1 = sc[8 * h + 2 * k + 1];
                const __m256i sv = _mm256_setr_epi16(s0, s0, s0, s0, s0, s0, s0, s0, s1, s1, s1, s1, s1, s1, s1, s1);
                acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p, sv));
            }
        }
        sum += d * (float)(hsum8(acc) - 32 * off);
    }
    return sum;
}

static float dot_row(int type, const uint8_t *w, const q8k_block *y, int nb)
{
    return type == T_Q6_K ? dot_q6k(w, y, nb) : dot_q4k(w, y, nb);
}

static long block_bytes(int type) { return type == T_Q6_K ? 210 : 144; }

/* y[r] (+)= W_r . x for up to three matrices sharing the quantized x
 * (KQuantGemv.Multi): rows of all targets in one dynamic-chunk loop */
typedef struct {
    int type, rows;
    const uint8_t *w;
    float *y;
    int accumulate;
} target;

static void gemv_multi(const q8k_block *xq, int cols, const target *t, int nt, int threads)
{
    const int nb = cols / 256;
    int total = 0;
    for (int i = 0; i < nt; i++) total += t[i].rows;
    int chunk = total / (threads * 16);
    if (chunk < 8) chunk = 8;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int c0 = 0; c0 < total; c0 += chunk) {
        for (int r = c0; r < c0 + chunk && r < total; r++) {
            int i = 0, rr = r;
            while (rr >= t[i].rows) rr -= t[i++].rows;
            const float v = dot_row(t[i].type, t[i].w + (long)rr * nb * block_bytes(t[i].type), xq, nb);
            t[i].y[rr] = t[i].accumulate ? t[i].y[rr] + v : v;
        }
    }
}

static void linear(const void *w, int type, int rows, int cols, const float *x, float *y, int acc, q8k_block *xq,
                   int threads)
{
    q8k_quantize(x, xq, cols);
    const target t = {type, rows, (const uint8_t *)w, y, acc};
    gemv_multi(xq, cols, &t, 1, threads);
}

int orc_cpu_q8k_gemv(int type, const void *w, int rows, int cols, const float *x, float *y, int accumulate,
                     int threads)
{
    if ((type != T_Q4_K && type != T_Q6_K) || cols % 256 != 0) return -1;
    q8k_block *xq = malloc(sizeof(q8k_block) * (cols / 256));
    if (!xq) return -1;
    linear(w, type, rows, cols, x, y, accumulate, xq, threads);
    free(xq);
    return 0;
}

int orc_cpu_decode_step(const orc_cpu_model *m, int token, int pos, float *logits, int threads)
{
    const int H = m->hidden, F = m->ffn, qd = m->heads * m->head_dim, kd = m->kv_heads * m->head_dim;
    /* the Q8_K buffer holds the widest projection input: hidden, ffn or the
       attention output (heads * head_dim, quantised for the o projection) */
    const int maxc = F > H ? (F > qd ? F : qd) : (H > qd ? H : qd);
    float *h = malloc(sizeof(float) * H), *n = malloc(sizeof(float) * H);
    float *q = malloc(sizeof(float) * qd), *k = malloc(sizeof(float) * kd), *v = malloc(sizeof(float) * kd);
    float *ao = malloc(sizeof(float) * qd), *g = malloc(sizeof(float) * F), *u = malloc(sizeof(float) * F);
    q8k_block *xq = malloc(sizeof(q8k_block) * (maxc / 256 + 1));
    int rc = -1;
    if (!h || !n || !q || !k || !v || !ao || !g || !u || !xq) goto out;
    {
        const long erb = (long)(H / 256) * block_bytes(m->embd_type);
        if (orc_dequant_row(m->embd_type, (const uint8_t *)m->embd + (long)token * erb, H, h) != 0) goto out;
    }
    for (int l = 0; l < m->layers; l++) {
        const orc_cpu_layer *L = &m->layer[l];
        orc_rmsnorm(h, L->attn_norm, n, 1, H, m->eps);
        q8k_quantize(n, xq, H);
        {
            const target t[3] = {{L->wq_type, qd, L->wq, q, 0}, {L->wk_type, kd, L->wk, k, 0},
                                 {L->wv_type, kd, L->wv, v, 0}};
            gemv_multi(xq, H, t, 3, threads);
        }
        orc_decode_attention(q, k, v, L->q_norm, L->k_norm, L->cache_k, L->cache_v, m->kv_dtype, m->heads,
                             m->kv_heads, m->head_dim, m->rope_dim, m->rope_base, m->eps, pos, ao, threads);
        linear(L->wo, L->wo_type, H, qd, ao, h, 1, xq, threads);
        orc_rmsnorm(h, L->ffn_norm, n, 1, H, m->eps);
        q8k_quantize(n, xq, H);
        {
            const target t[2] = {{L->wg_type, F, L->wg, g, 0}, {L->wu_type, F, L->wu, u, 0}};
            gemv_multi(xq, H, t, 2, threads);
        }
        for (int i = 0; i < F; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i]; /* Ops.SiLUMul */
        linear(L->wd, L->wd_type, H, F, g, h, 1, xq, threads);
    }
    orc_rmsnorm(h, m->out_norm, n, 1, H, m->eps);
    linear(m->out, m->out_type, m->vocab, H, n, logits, 0, xq, threads);
    rc = 0;
out:
    free(h); free(n); free(q); free(k); free(v); free(ao); free(g); free(u); free(xq);
    return rc;
}
