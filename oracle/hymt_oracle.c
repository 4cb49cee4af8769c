/*
 * hymt_oracle.c -- CPU restatement of HyMT2Sharp's attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the thing
 * measured or shipped.  See hymt_oracle.h for the list of functions, the
 * reference lines each follows and the checks that pin each of them.
 *
 * Built with -ffp-contract=off so that a*b+c stays two roundings where the
 * reference writes two operations, and fmaf() appears exactly where the
 * reference calls Fma.MultiplyAdd.
 */
#include "hymt_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Ops.cs:664-665: RNE by integer add, no NaN special case. */
uint16_t orc_f32_to_bf16(float x)
{
    uint32_t bits = f2u(x);
    return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

/* Ops.cs:688 */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE-754 binary16, round to nearest, ties to even; overflow -> inf, NaN kept quiet. */
uint16_t orc_f32_to_f16(float x)
{
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ax = u & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? (0x200u | ((ax >> 13) & 0x3FFu)) : 0u));
    if (ax >= 0x477FF000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax >= 0x38800000u) { /* normal half: rebias exponent 127 -> 15, round 13 bits */
        uint32_t r = ax - (112u << 23);
        return (uint16_t)(sign | ((r + 0xFFFu + ((r >> 13) & 1u)) >> 13));
    }
    /* half subnormal: value * 2^24 rounded to an integer in [0, 1024] */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7FFFFFu) | (e ? 0x800000u : 0u);
    int shift = (e ? 126 - (int)e : 125);
    if (shift >= 32)
        return (uint16_t)sign;
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u)))
        q++;
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1F)
        return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_convert(const float *src, void *dst, long n, int dtype)
{
    if (dtype == ORC_F32) {
        memcpy(dst, src, (size_t)n * 4);
    } else if (dtype == ORC_BF16) {
        uint16_t *d = (uint16_t *)dst;
        for (long i = 0; i < n; i++) d[i] = orc_f32_to_bf16(src[i]);
    } else {
        uint16_t *d = (uint16_t *)dst;
        for (long i = 0; i < n; i++) d[i] = orc_f32_to_f16(src[i]);
    }
}

float orc_load(const void *base, long i, int dtype)
{
    if (dtype == ORC_F32) return ((const float *)base)[i];
    if (dtype == ORC_BF16) return orc_bf16_to_f32(((const uint16_t *)base)[i]);
    return orc_f16_to_f32(((const uint16_t *)base)[i]);
}

/* widen 8 consecutive cache elements (LoadBf16x8, Ops.cs:702-703) */
static inline void load8(const void *base, long i, int dtype, float *o)
{
    if (dtype == ORC_F32) {
        memcpy(o, (const float *)base + i, 32);
    } else if (dtype == ORC_BF16) {
        const uint16_t *p = (const uint16_t *)base + i;
        for (int l = 0; l < 8; l++) o[l] = u2f((uint32_t)p[l] << 16);
    } else {
        /* exact widening; F16C does it in one instruction (vcvtph2ps) */
        __m128i h = _mm_loadu_si128((const __m128i *)((const uint16_t *)base + i));
        _mm256_storeu_ps(o, _mm256_cvtph_ps(h));
    }
}

/* ------------------------------------------------------------------------ */
/* horizontal reductions of a Vector256<float>                               */
/* ------------------------------------------------------------------------ */

/* VecDotQ4K.HorizontalSum (VecDotQ4K.cs:383-389) */
static inline float hsum8(const float *a)
{
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

/* Ops.HorizontalSum4 (Ops.cs:648-654): element r of the result is the sum of
 * vector r, in the vhaddps association order. */
static inline float hsum4_elem(const float *a)
{
    float lo = (a[0] + a[1]) + (a[2] + a[3]);
    float hi = (a[4] + a[5]) + (a[6] + a[7]);
    return lo + hi;
}

/* ------------------------------------------------------------------------ */
/* FastExp                                                                   */
/* ------------------------------------------------------------------------ */

/* FastExp.ExpAvx2 (FastExp.cs:15-46), lane by lane.  The reference takes the
 * non-overflow result for all 8 lanes when no lane overflows; the per-lane
 * select below gives the same value in every lane. */
void orc_fast_exp8(const float *x, float *y)
{
    for (int l = 0; l < 8; l++) {
        const float r = 12582912.0f;
        float z = fmaf(x[l], 1.4426950216293335f, r);
        float n = z - r;
        /* Fma.MultiplyAddNegated(a, b, c) = -(a*b) + c, one rounding */
        float b = fmaf(-n, 1.4286067655086517e-6f, fmaf(-n, 0.693145751953125f, x[l]));
        uint32_t e = f2u(z) << 23;
        float k = u2f(e + f2u(1.0f));
        float nabs = fabsf(n);
        int overflow = nabs > 126.0f;
        float u = b * b;
        float j = fmaf(fmaf(fmaf(0.008301135152578354f, b, 0.04190601035952568f), u,
                            fmaf(0.166665181517601f, b, 0.4999998211860657f)),
                       u, 0.9999998211860657f * b);
        if (!overflow) {
            y[l] = fmaf(j, k, k);
            continue;
        }
        uint32_t g = (n <= 0.0f) ? 0x82000000u : 0u;
        float s1 = u2f(g + 0x7F000000u);
        float s2 = u2f(e - g);
        if (nabs > 192.0f)
            y[l] = s1 * s1;
        else
            y[l] = fmaf(s2, j, s2) * s1;
    }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm                                                                   */
/* ------------------------------------------------------------------------ */

/* Ops.RmsNormRange (Ops.cs:29-90), AVX path: 8-lane FMA sum of squares,
 * HorizontalSum, scalar tail, then x*scale*w. */
void orc_rmsnorm(const float *x, const float *weight, float *y, int rows, int dim, float eps)
{
    for (int r = 0; r < rows; r++) {
        const float *src = x + (long)r * dim;
        float *dst = y + (long)r * dim;
        float acc[8] = {0};
        int i = 0;
        for (; i <= dim - 8; i += 8)
            for (int l = 0; l < 8; l++) acc[l] = fmaf(src[i + l], src[i + l], acc[l]);
        float sum = hsum8(acc);
        for (; i < dim; i++) sum += src[i] * src[i];
        float scale = 1.0f / sqrtf(sum / (float)dim + eps);
        for (i = 0; i < dim; i++) {
            float v = src[i] * scale;
            if (weight) v = v * weight[i];
            dst[i] = v;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                      */
/* ------------------------------------------------------------------------ */

static void rope_freqs(int half, float base, float *freqs)
{
    /* Ops.cs:176-177 */
    for (int i = 0; i < half; i++) freqs[i] = 1.0f / powf(base, (float)i / (float)half);
}

void orc_rope_table(int half, float base, int cap, float *cos_out, float *sin_out)
{
    float *freqs = (float *)malloc(sizeof(float) * (size_t)half);
    rope_freqs(half, base, freqs);
    /* Ops.cs:180-188: angle = pos * freq in fp32 */
    for (int pos = 0; pos < cap; pos++)
        for (int i = 0; i < half; i++) {
            float angle = (float)pos * freqs[i];
            cos_out[(long)pos * half + i] = cosf(angle);
            sin_out[(long)pos * half + i] = sinf(angle);
        }
    free(freqs);
}

/* Ops.RopeRange (Ops.cs:120-168).  Table rows are generated for the
 * positions in use only; each is the same value EnsureRopeTable stores. */
void orc_neox_rope(float *x, int tokens, int heads, int head_dim, int rope_dim, int start_pos,
                   float base)
{
    int half = rope_dim / 2;
    float *freqs = (float *)malloc(sizeof(float) * (size_t)half);
    float *c = (float *)malloc(sizeof(float) * (size_t)half);
    float *s = (float *)malloc(sizeof(float) * (size_t)half);
    rope_freqs(half, base, freqs);
    for (int t = 0; t < tokens; t++) {
        int pos = start_pos + t;
        for (int i = 0; i < half; i++) {
            float angle = (float)pos * freqs[i];
            c[i] = cosf(angle);
            s[i] = sinf(angle);
        }
        for (int h = 0; h < heads; h++) {
            float *row = x + ((long)t * heads + h) * head_dim;
            for (int i = 0; i < half; i++) {
                float x0 = row[i], x1 = row[i + half];
                row[i] = x0 * c[i] - x1 * s[i];
                row[i + half] = x0 * s[i] + x1 * c[i];
            }
        }
    }
    free(freqs);
    free(c);
    free(s);
}

/* ------------------------------------------------------------------------ */
/* softmax                                                                   */
/* ------------------------------------------------------------------------ */

/* Ops.SoftmaxRow (Ops.cs:224-325), AVX2+FMA path for n >= 8, scalar below. */
void orc_softmax_row(float *row, int n)
{
    int i = 0;
    float max, sum;
    if (n >= 8) {
        float vmax[8];
        for (int l = 0; l < 8; l++) vmax[l] = -80.0f;
        for (; i <= n - 8; i += 8)
            for (int l = 0; l < 8; l++) vmax[l] = row[i + l] > vmax[l] ? row[i + l] : vmax[l];
        max = vmax[0];
        for (int l = 1; l < 8; l++) if (vmax[l] > max) max = vmax[l];
        for (; i < n; i++) if (row[i] > max) max = row[i];

        float vsum[8] = {0};
        i = 0;
        for (; i <= n - 8; i += 8) {
            float sh[8], e[8];
            for (int l = 0; l < 8; l++) {
                float d = row[i + l] - max;
                sh[l] = d > -80.0f ? d : -80.0f;
            }
            orc_fast_exp8(sh, e);
            for (int l = 0; l < 8; l++) {
                row[i + l] = e[l];
                vsum[l] = vsum[l] + e[l];
            }
        }
        sum = hsum8(vsum);
        for (; i < n; i++) {
            float e = expf(fmaxf(row[i] - max, -80.0f));
            row[i] = e;
            sum += e;
        }
    } else {
        max = -80.0f;
        for (i = 0; i < n; i++) if (row[i] > max) max = row[i];
        sum = 0;
        for (i = 0; i < n; i++) {
            float e = expf(fmaxf(row[i] - max, -80.0f));
            row[i] = e;
            sum += e;
        }
    }
    float inv = sum > 0 ? 1.0f / sum : 0.0f;
    for (i = 0; i < n; i++) row[i] = row[i] * inv;
}

static inline int worker_count(int threads, int count)
{
    int w = threads < 1 ? 1 : threads;
    return w < count ? w : count; /* CpuThreadPool.cs:60: min(ThreadCount, count) */
}

/* Ops.SoftmaxCausal (Ops.cs:198-221) */
void orc_softmax_causal(float *scores, int heads, int q_len, int kv_len, int start_pos, int threads)
{
    int workers = worker_count(threads, heads);
#pragma omp parallel for num_threads(workers) schedule(static, 1)
    for (int w = 0; w < workers; w++) {
        int begin = heads * w / workers, end = heads * (w + 1) / workers;
        for (int h = begin; h < end; h++)
            for (int q = 0; q < q_len; q++) {
                float *row = scores + ((long)h * q_len + q) * kv_len;
                int allowed = kv_len < start_pos + q + 1 ? kv_len : start_pos + q + 1;
                orc_softmax_row(row, allowed);
                for (int t = allowed; t < kv_len; t++) row[t] = 0.0f;
            }
    }
}

/* ------------------------------------------------------------------------ */
/* dot products over cache rows                                              */
/* ------------------------------------------------------------------------ */

/* Ops.DotBf16 (Ops.cs:707-744): two 8-lane accumulators over 16-wide steps,
 * an 8-wide step, HorizontalSum(acc0+acc1), scalar tail. */
static float dot_row(const float *a, const void *b, long boff, int n, int dtype)
{
    float acc0[8] = {0}, acc1[8] = {0}, v[8];
    int i = 0;
    for (; i <= n - 16; i += 16) {
        load8(b, boff + i, dtype, v);
        for (int l = 0; l < 8; l++) acc0[l] = fmaf(a[i + l], v[l], acc0[l]);
        load8(b, boff + i + 8, dtype, v);
        for (int l = 0; l < 8; l++) acc1[l] = fmaf(a[i + 8 + l], v[l], acc1[l]);
    }
    for (; i <= n - 8; i += 8) {
        load8(b, boff + i, dtype, v);
        for (int l = 0; l < 8; l++) acc0[l] = fmaf(a[i + l], v[l], acc0[l]);
    }
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = acc0[l] + acc1[l];
    float sum = hsum8(s);
    for (; i < n; i++) sum += a[i] * orc_load(b, boff + i, dtype);
    return sum;
}

/* Ops.DotBf16x4 (Ops.cs:748-816): four rows sharing each q load; result * scale. */
static void dot_x4(const float *q, const void *k, long off0, long stride, int n, int dtype,
                   float *dst, float scale)
{
    float acc[4][8] = {{0}}, v[8];
    int i = 0;
    for (; i <= n - 8; i += 8)
        for (int r = 0; r < 4; r++) {
            load8(k, off0 + r * stride + i, dtype, v);
            for (int l = 0; l < 8; l++) acc[r][l] = fmaf(q[i + l], v[l], acc[r][l]);
        }
    float s[4];
    for (int r = 0; r < 4; r++) s[r] = hsum8(acc[r]);
    for (; i < n; i++)
        for (int r = 0; r < 4; r++) s[r] += q[i] * orc_load(k, off0 + r * stride + i, dtype);
    for (int r = 0; r < 4; r++) dst[r] = s[r] * scale;
}

/* Ops.Dot2x4Bf16 (Ops.cs:820-854): two q rows x four K rows, HorizontalSum4. */
static void dot_2x4(const float *q0, const float *q1, const void *k, long off0, long stride, int n,
                    int dtype, float *dst0, float *dst1, float scale)
{
    float a0[4][8] = {{0}}, a1[4][8] = {{0}}, v[8];
    for (int i = 0; i < n; i += 8)
        for (int r = 0; r < 4; r++) {
            load8(k, off0 + r * stride + i, dtype, v);
            for (int l = 0; l < 8; l++) {
                a0[r][l] = fmaf(q0[i + l], v[l], a0[r][l]);
                a1[r][l] = fmaf(q1[i + l], v[l], a1[r][l]);
            }
        }
    for (int r = 0; r < 4; r++) {
        dst0[r] = hsum4_elem(a0[r]) * scale;
        dst1[r] = hsum4_elem(a1[r]) * scale;
    }
}

/* Ops.Axpy64Bf16 (Ops.cs:923-955): dst[0..64) = sum_kt w[kt] * v[kt][0..64),
 * one FMA chain per element in kt order. */
static void axpy64(const float *w, const void *v, long off0, long stride, int count, int dtype,
                   float *dst)
{
    float a[64] = {0}, x[8];
    for (int kt = 0; kt < count; kt++) {
        float wv = w[kt];
        long row = off0 + (long)kt * stride;
        for (int c = 0; c < 8; c++) {
            load8(v, row + 8 * c, dtype, x);
            for (int l = 0; l < 8; l++) a[8 * c + l] = fmaf(wv, x[l], a[8 * c + l]);
        }
    }
    memcpy(dst, a, sizeof(a));
}

/* Head-dim tail of AttentionDecode/AttentionCombine (Ops.cs:518-524, 576-586). */
static void axpy_tail(const float *w, const void *v, long off0, long stride, int count, int dtype,
                      float *dst, int n)
{
    for (int i = 0; i < n; i++) dst[i] = 0.0f;
    for (int kt = 0; kt < count; kt++)
        for (int i = 0; i < n; i++)
            dst[i] += w[kt] * orc_load(v, off0 + (long)kt * stride + i, dtype);
}

/* ------------------------------------------------------------------------ */
/* attention                                                                 */
/* ------------------------------------------------------------------------ */

void orc_attention_scores(const float *q, const void *cache_k, int kv_dtype, float *scores,
                          int heads, int kv_heads, int head_dim, int q_len, int kv_len, int q_dim,
                          int kv_stride, float scale, int start_pos, int threads)
{
    int group = heads / kv_heads;
    int workers = worker_count(threads, heads);
#pragma omp parallel for num_threads(workers) schedule(static, 1)
    for (int w = 0; w < workers; w++) {
        int begin = heads * w / workers, end = heads * (w + 1) / workers;
        for (int h = begin; h < end; h++) {
            int kvh = h / group;
            long kbase = (long)kvh * head_dim;
            int qt = 0;
            if ((head_dim & 7) == 0) {
                /* Ops.cs:388-404: row pairs; row qt's extra score past its causal
                 * bound lands in the tail SoftmaxCausal zeroes. */
                for (; qt + 1 < q_len; qt += 2) {
                    const float *q0 = q + (long)qt * q_dim + (long)h * head_dim;
                    const float *q1 = q0 + q_dim;
                    float *row0 = scores + ((long)h * q_len + qt) * kv_len;
                    float *row1 = row0 + kv_len;
                    int allowed = kv_len < start_pos + qt + 2 ? kv_len : start_pos + qt + 2;
                    int kt = 0;
                    for (; kt + 3 < allowed; kt += 4)
                        dot_2x4(q0, q1, cache_k, kbase + (long)kt * kv_stride, kv_stride, head_dim,
                                kv_dtype, row0 + kt, row1 + kt, scale);
                    for (; kt < allowed; kt++) {
                        long off = kbase + (long)kt * kv_stride;
                        row0[kt] = dot_row(q0, cache_k, off, head_dim, kv_dtype) * scale;
                        row1[kt] = dot_row(q1, cache_k, off, head_dim, kv_dtype) * scale;
                    }
                }
            }
            for (; qt < q_len; qt++) {
                const float *qh = q + (long)qt * q_dim + (long)h * head_dim;
                float *row = scores + ((long)h * q_len + qt) * kv_len;
                int allowed = kv_len < start_pos + qt + 1 ? kv_len : start_pos + qt + 1;
                int kt = 0;
                for (; kt + 3 < allowed; kt += 4)
                    dot_x4(qh, cache_k, kbase + (long)kt * kv_stride, kv_stride, head_dim, kv_dtype,
                           row + kt, scale);
                for (; kt < allowed; kt++)
                    row[kt] = dot_row(qh, cache_k, kbase + (long)kt * kv_stride, head_dim,
                                      kv_dtype) * scale;
            }
        }
    }
}

static void combine_row(const float *row, const void *cache_v, long vbase, int kv_stride,
                        int allowed, int kv_dtype, int head_dim, float *out_h)
{
    int d = 0;
    for (; d + 63 < head_dim; d += 64)
        axpy64(row, cache_v, vbase + d, kv_stride, allowed, kv_dtype, out_h + d);
    if (d < head_dim)
        axpy_tail(row, cache_v, vbase + d, kv_stride, allowed, kv_dtype, out_h + d, head_dim - d);
}

void orc_attention_decode(const float *q, const void *cache_k, const void *cache_v, int kv_dtype,
                          float *scores, float *output, int heads, int kv_heads, int head_dim,
                          int kv_len, int kv_stride, float scale, int start_pos, int threads)
{
    int group = heads / kv_heads;
    int workers = worker_count(threads, heads);
#pragma omp parallel for num_threads(workers) schedule(static, 1)
    for (int w = 0; w < workers; w++) {
        int begin = heads * w / workers, end = heads * (w + 1) / workers;
        for (int h = begin; h < end; h++) {
            int kvh = h / group;
            const float *qh = q + (long)h * head_dim;
            long kbase = (long)kvh * head_dim, vbase = (long)kvh * head_dim;
            float *row = scores + (long)h * kv_len;
            int allowed = kv_len < start_pos + 1 ? kv_len : start_pos + 1;
            int kt = 0;
            for (; kt + 3 < allowed; kt += 4)
                dot_x4(qh, cache_k, kbase + (long)kt * kv_stride, kv_stride, head_dim, kv_dtype,
                       row + kt, scale);
            for (; kt < allowed; kt++)
                row[kt] = dot_row(qh, cache_k, kbase + (long)kt * kv_stride, head_dim, kv_dtype) *
                          scale;
            orc_softmax_row(row, allowed);
            combine_row(row, cache_v, vbase, kv_stride, allowed, kv_dtype, head_dim,
                        output + (long)h * head_dim);
        }
    }
}

void orc_attention_combine(const void *cache_v, int kv_dtype, const float *scores, float *output,
                           int heads, int kv_heads, int head_dim, int q_len, int kv_len, int q_dim,
                           int kv_stride, int start_pos, int threads)
{
    int group = heads / kv_heads;
    int workers = worker_count(threads, heads);
#pragma omp parallel for num_threads(workers) schedule(static, 1)
    for (int w = 0; w < workers; w++) {
        int begin = heads * w / workers, end = heads * (w + 1) / workers;
        for (int h = begin; h < end; h++) {
            int kvh = h / group;
            long vbase = (long)kvh * head_dim;
            for (int qt = 0; qt < q_len; qt++) {
                const float *row = scores + ((long)h * q_len + qt) * kv_len;
                int allowed = kv_len < start_pos + qt + 1 ? kv_len : start_pos + qt + 1;
                combine_row(row, cache_v, vbase, kv_stride, allowed, kv_dtype, head_dim,
                            output + (long)qt * q_dim + (long)h * head_dim);
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* layer-level orchestration                                                 */
/* ------------------------------------------------------------------------ */

static size_t dtype_size(int dtype) { return dtype == ORC_F32 ? 4 : 2; }

void orc_decode_attention(float *q, float *k, const float *v, const float *qnw, const float *knw,
                          void *cache_k, void *cache_v, int kv_dtype, int heads, int kv_heads,
                          int head_dim, int rope_dim, float rope_base, float eps, int start,
                          float *out, int threads)
{
    int k_dim = kv_heads * head_dim;
    /* HunyuanDenseModel.Decode.cs:80-88 */
    orc_neox_rope(q, 1, heads, head_dim, rope_dim, start, rope_base);
    orc_neox_rope(k, 1, kv_heads, head_dim, rope_dim, start, rope_base);
    if (qnw) orc_rmsnorm(q, qnw, q, heads, head_dim, eps);
    if (knw) orc_rmsnorm(k, knw, k, kv_heads, head_dim, eps);
    size_t es = dtype_size(kv_dtype);
    orc_convert(k, (char *)cache_k + (size_t)start * k_dim * es, k_dim, kv_dtype);
    orc_convert(v, (char *)cache_v + (size_t)start * k_dim * es, k_dim, kv_dtype);
    /* Decode.cs:90-95 */
    int kv_len = start + 1;
    float scale = 1.0f / sqrtf((float)head_dim);
    float *sc = (float *)malloc(sizeof(float) * (size_t)heads * kv_len);
    orc_attention_decode(q, cache_k, cache_v, kv_dtype, sc, out, heads, kv_heads, head_dim, kv_len,
                         k_dim, scale, start, threads);
    free(sc);
}

void orc_prefill_attention(float *q, float *k, const float *v, const float *qnw, const float *knw,
                           void *cache_k, void *cache_v, int kv_dtype, int heads, int kv_heads,
                           int head_dim, int rope_dim, float rope_base, float eps, int start,
                           int seq, float *out, int threads)
{
    int q_dim = heads * head_dim, k_dim = kv_heads * head_dim;
    /* HunyuanDenseModel.Prefill.cs:53-61 */
    orc_neox_rope(q, seq, heads, head_dim, rope_dim, start, rope_base);
    orc_neox_rope(k, seq, kv_heads, head_dim, rope_dim, start, rope_base);
    if (qnw) orc_rmsnorm(q, qnw, q, seq * heads, head_dim, eps);
    if (knw) orc_rmsnorm(k, knw, k, seq * kv_heads, head_dim, eps);
    size_t es = dtype_size(kv_dtype);
    orc_convert(k, (char *)cache_k + (size_t)start * k_dim * es, (long)seq * k_dim, kv_dtype);
    orc_convert(v, (char *)cache_v + (size_t)start * k_dim * es, (long)seq * k_dim, kv_dtype);
    /* Prefill.cs:63-83 */
    int kv_len = start + seq;
    float scale = 1.0f / sqrtf((float)head_dim);
    float *sc = (float *)malloc(sizeof(float) * (size_t)heads * seq * kv_len);
    orc_attention_scores(q, cache_k, kv_dtype, sc, heads, kv_heads, head_dim, seq, kv_len, q_dim,
                         k_dim, scale, start, threads);
    orc_softmax_causal(sc, heads, seq, kv_len, start, threads);
    orc_attention_combine(cache_v, kv_dtype, sc, out, heads, kv_heads, head_dim, seq, kv_len, q_dim,
                          k_dim, start, threads);
    free(sc);
}

void orc_forward_prefill_attention(float *q, float *k, const float *v, const float *qnw,
                                   const float *knw, void *cache_k, void *cache_v, int kv_dtype,
                                   int heads, int kv_heads, int head_dim, int rope_dim,
                                   float rope_base, float eps, int start, int seq, float *out,
                                   int threads)
{
    const int chunk = 1024; /* HunyuanDenseModel.cs:348-355 */
    int q_dim = heads * head_dim, k_dim = kv_heads * head_dim;
    for (int off = 0; off < seq; off += chunk) {
        int n = seq - off < chunk ? seq - off : chunk;
        orc_prefill_attention(q + (long)off * q_dim, k + (long)off * k_dim, v + (long)off * k_dim,
                              qnw, knw, cache_k, cache_v, kv_dtype, heads, kv_heads, head_dim,
                              rope_dim, rope_base, eps, start + off, n, out + (long)off * q_dim,
                              threads);
    }
}

void orc_attention_f64(const float *q, const float *cache_k, const float *cache_v, int heads,
                       int kv_heads, int head_dim, int start, int seq, double scale, double *out)
{
    int group = heads / kv_heads;
    int q_dim = heads * head_dim, k_dim = kv_heads * head_dim;
    int kv_len = start + seq;
    double *p = (double *)malloc(sizeof(double) * (size_t)kv_len);
    for (int t = 0; t < seq; t++)
        for (int h = 0; h < heads; h++) {
            int kvh = h / group, allowed = start + t + 1;
            const float *qh = q + (long)t * q_dim + (long)h * head_dim;
            double m = -1e300, sum = 0;
            for (int j = 0; j < allowed; j++) {
                const float *kr = cache_k + (long)j * k_dim + (long)kvh * head_dim;
                double s = 0;
                for (int d = 0; d < head_dim; d++) s += (double)qh[d] * (double)kr[d];
                p[j] = s * scale;
                if (p[j] > m) m = p[j];
            }
            for (int j = 0; j < allowed; j++) { p[j] = exp(p[j] - m); sum += p[j]; }
            double *o = out + (long)t * q_dim + (long)h * head_dim;
            for (int d = 0; d < head_dim; d++) o[d] = 0;
            for (int j = 0; j < allowed; j++) {
                const float *vr = cache_v + (long)j * k_dim + (long)kvh * head_dim;
                for (int d = 0; d < head_dim; d++) o[d] += p[j] / sum * (double)vr[d];
            }
        }
    free(p);
}
