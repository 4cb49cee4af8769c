/*
 * hymt_oracle.h -- CPU restatement of HyMT2Sharp's attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path in hymt2sharp_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never links it and
 * never falls back to it.
 *
 * Every function restates one function of the reference (C#, .NET 10) in
 * plain C, following the cited file:line of /root/reference/src/HyMT2Sharp.
 * The reference cannot be compiled here (no .NET), so nothing is built from
 * its sources.  Accumulation orders follow the reference's AVX2+FMA tier
 * (Simd.cs:25-28): 8-lane FMA accumulators, then the same horizontal-sum
 * order, so results track the reference to a few ulp.  Bit equality with the
 * .NET JIT is not claimed (MathF.* are libm calls there as here).
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   orc_f32_to_bf16 / orc_bf16_to_f32  exhaustive + independent RNE model
 *   orc_f32_to_f16  / orc_f16_to_f32   numpy float16 (IEEE RNE), all 2^16 halves
 *   orc_fast_exp8                      FastExpTests tolerance 2e-5 vs libm exp
 *   orc_rope_table / orc_neox_rope     fp64 closed form, pos 0 identity,
 *                                      pair-norm invariance
 *   orc_rmsnorm                        fp64 closed form, rms(y/g)=1
 *   orc_softmax_row / _causal          AttentionTests.SoftmaxCausal metric 2e-3,
 *                                      row sums, masked zeros, -80 floor rows
 *   orc_attention_scores / _combine    AttentionTests.ScoresAndCombine shapes
 *                                      and tolerances (5e-5 / 5e-4)
 *   orc_attention_decode               fp64 brute force, all-equal K -> mean V,
 *                                      dominant logit -> that V row
 *   orc_decode_attention /
 *   orc_prefill_attention              decode(p) == prefill row p, chunked ==
 *                                      monolithic, committed numpy-fp64 fixtures
 */
#ifndef HYMT_ORACLE_H
#define HYMT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KV storage dtypes; the values equal hymt_dtype in include/hymt_hip.h. */
#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2

/* Ops.cs:664-665 (ConvertToBf16) and Ops.cs:688 (Bf16ToF32). */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
/* IEEE binary16 round-to-nearest-even, as (Half)x in VulkanBackend.cs:895-903. */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
/* Ops.ConvertToBf16 (Ops.cs:658-680) generalised to the three cache dtypes. */
void orc_convert(const float *src, void *dst, long n, int dtype);
/* Element i of a cache of the given dtype, widened to fp32. */
float orc_load(const void *base, long i, int dtype);

/* FastExp.ExpAvx2 (FastExp.cs:15-46), one call = the 8 lanes of a Vector256. */
void orc_fast_exp8(const float *x, float *y);

/* Ops.RmsNorm / RmsNormRange (Ops.cs:12-90).  weight may be NULL. */
void orc_rmsnorm(const float *x, const float *weight, float *y, int rows, int dim, float eps);

/* Ops.EnsureRopeTable (Ops.cs:170-195): rows [0, cap) of the cos/sin tables. */
void orc_rope_table(int half, float base, int cap, float *cos_out, float *sin_out);
/* Ops.NeoXRoPE / RopeRange (Ops.cs:98-168), in place on [tokens][heads][head_dim]. */
void orc_neox_rope(float *x, int tokens, int heads, int head_dim, int rope_dim, int start_pos,
                   float base);

/* Ops.SoftmaxRow (Ops.cs:224-325) and Ops.SoftmaxCausal (Ops.cs:198-221). */
void orc_softmax_row(float *row, int n);
void orc_softmax_causal(float *scores, int heads, int q_len, int kv_len, int start_pos,
                        int threads);

/* Ops.AttentionScores (Ops.cs:359-455). */
void orc_attention_scores(const float *q, const void *cache_k, int kv_dtype, float *scores,
                          int heads, int kv_heads, int head_dim, int q_len, int kv_len, int q_dim,
                          int kv_stride, float scale, int start_pos, int threads);
/* Ops.AttentionDecode (Ops.cs:462-532). */
void orc_attention_decode(const float *q, const void *cache_k, const void *cache_v, int kv_dtype,
                          float *scores, float *output, int heads, int kv_heads, int head_dim,
                          int kv_len, int kv_stride, float scale, int start_pos, int threads);
/* Ops.AttentionCombine (Ops.cs:535-595). */
void orc_attention_combine(const void *cache_v, int kv_dtype, const float *scores, float *output,
                           int heads, int kv_heads, int head_dim, int q_len, int kv_len, int q_dim,
                           int kv_stride, int start_pos, int threads);

/*
 * HunyuanDenseModel.DecodeAttention (HunyuanDenseModel.Decode.cs:64-101),
 * attention part: RoPE q,k at `start` -> RMSNorm q,k -> append k,v rounded to
 * the cache dtype at row `start` -> AttentionDecode over [0, start].
 * q [heads*head_dim] and k [kv_heads*head_dim] are modified in place exactly
 * as in the reference; v is read only.  qnw/knw NULL skips that norm (the
 * reference always normalises; NULL exists for configs that name no norm).
 * cache_k/cache_v: flat [cap][kv_heads*head_dim] caches of kv_dtype.
 */
void orc_decode_attention(float *q, float *k, const float *v, const float *qnw, const float *knw,
                          void *cache_k, void *cache_v, int kv_dtype, int heads, int kv_heads,
                          int head_dim, int rope_dim, float rope_base, float eps, int start,
                          float *out, int threads);

/*
 * HunyuanDenseModel.PrefillAttention (HunyuanDenseModel.Prefill.cs:38-89),
 * attention part, for one chunk of `seq` tokens at `start`.  Same contract
 * as orc_decode_attention with q [seq][heads*head_dim], k,v
 * [seq][kv_heads*head_dim], out [seq][heads*head_dim].
 */
void orc_prefill_attention(float *q, float *k, const float *v, const float *qnw, const float *knw,
                           void *cache_k, void *cache_v, int kv_dtype, int heads, int kv_heads,
                           int head_dim, int rope_dim, float rope_base, float eps, int start,
                           int seq, float *out, int threads);

/*
 * HunyuanDenseModel.Forward prefill chunking (HunyuanDenseModel.cs:342-355):
 * a prompt longer than 1024 tokens runs as consecutive 1024-token chunks,
 * each attending over the cache the earlier chunks wrote.
 */
void orc_forward_prefill_attention(float *q, float *k, const float *v, const float *qnw,
                                   const float *knw, void *cache_k, void *cache_v, int kv_dtype,
                                   int heads, int kv_heads, int head_dim, int rope_dim,
                                   float rope_base, float eps, int start, int seq, float *out,
                                   int threads);

/*
 * fp64 brute-force causal GQA attention over an fp32 copy of the cache
 * (mirrors MetalGemvMicro.RunAttn, MetalGemvMicro.cs:292-384): for query row
 * t at absolute position start+t, keys [0, start+t] are visible.  Used only
 * to pin the fp32 restatements above.
 */
void orc_attention_f64(const float *q, const float *cache_k, const float *cache_v, int heads,
                       int kv_heads, int head_dim, int start, int seq, double scale, double *out);

/*
 * Quantized weight rows (hymt_quant.c): GGUF type codes 0 F32, 1 F16, 8 Q8_0,
 * 12 Q4_K, 14 Q6_K, 40 Q2_0C, 43 STQ1_0 (GgmlTensorType.cs).  Pinned by the
 * round trips of independent encoders in tests/test_quant_oracle.py.
 */
long orc_row_bytes(int type, int n);
int orc_dequant_row(int type, const void *row, int n, float *y);
int orc_gemv(int type, const void *w, int rows, int cols, const float *x, float *y, int accumulate);

/*
 * The reference's CPU decode step (cpu_decode.c): projections over Q8_K-
 * quantized activations (Q8K.cs, VecDotQ4K.cs, Q6K.cs, KQuantGemv.cs) around
 * orc_decode_attention, in the order of HunyuanDenseModel.Decode.cs:30-101.
 * The CPU baseline bench.py times; pinned against orc_gemv and the fp64 model
 * step within the Q8_K quantisation bound (tests/test_cpu_decode_port.py).
 * Weights are GGUF blocks of Q4_K (12) or Q6_K (14); the cache is kv_dtype.
 */
typedef struct {
    const void *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    int wq_type, wk_type, wv_type, wo_type, wg_type, wu_type, wd_type;
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
    void *cache_k, *cache_v;  /* [cap][kv_heads*head_dim] */
} orc_cpu_layer;

typedef struct {
    int layers, hidden, ffn, vocab, heads, kv_heads, head_dim, rope_dim, kv_dtype;
    float eps, rope_base;
    const void *embd;        /* token embedding, embd_type blocks */
    int embd_type;
    const void *out;         /* output projection (the embedding when tied) */
    int out_type;
    const float *out_norm;
    const orc_cpu_layer *layer;
} orc_cpu_model;

/* y (+)= W . q8k(x) with W Q4_K or Q6_K, rows over `threads` threads */
int orc_cpu_q8k_gemv(int type, const void *w, int rows, int cols, const float *x, float *y, int accumulate,
                     int threads);
/* one decode step at `pos` for `token`: logits[vocab]; appends to the caches */
int orc_cpu_decode_step(const orc_cpu_model *m, int token, int pos, float *logits, int threads);

#ifdef __cplusplus
}
#endif

#endif
