/*
 * hymt_hip.h -- C ABI of libhymt_hip.so, the MI355X (gfx950) attention path
 * for HyMT2Sharp.
 *
 * The library is what a C# `HipBackend : IComputeBackend` binds through
 * P/Invoke ([LibraryImport("hymt_hip")], the same pattern as Vk.cs:10-25 in
 * the reference).  It owns the HIP device, one in-order stream, a paged
 * device-resident K/V cache per layer and the attention kernels:
 * RoPE + per-head Q/K RMSNorm + KV append + GQA softmax(QK^T)V, for causal
 * prefill and single-token decode.
 *
 * Conventions
 *  - Every function returns an int status (hymt_status); 0 is success.  A
 *    failing call leaves a message for hymt_last_error() in thread-local
 *    storage.  The library never aborts the process.
 *  - All work is ordered on the context's single stream.  Calls on one
 *    context must come from one thread at a time, as the reference's model
 *    is not thread-safe (README_EN.md:118).
 *  - Arguments are plain pointers, ints and floats (blittable for P/Invoke).
 *    Without HYMT_FLAG_DEVICE_PTRS, tensor pointers are host memory and the
 *    call returns when the result is in host memory.  With it they are
 *    device pointers (hymt_dev_alloc) and the call only enqueues work.
 *  - Layouts follow the reference: q [seq][heads*head_dim],
 *    k/v [seq][kv_heads*head_dim], out [seq][heads*head_dim], fp32, rows of
 *    the model's flat caches are pos*kv_stride (IComputeBackend.cs:31-38).
 */
#ifndef HYMT_HIP_H
#define HYMT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HYMT_ABI_VERSION 1

/* Status codes.  The C# binding maps them onto the exceptions the reference
 * backends throw (VulkanBackend.cs:80-89, 893-894, 1088-1089; Vk.cs:30-34). */
typedef enum hymt_status {
    HYMT_OK = 0,
    HYMT_E_ARG = 1,         /* ArgumentException: bad pointer, size or index      */
    HYMT_E_UNSUPPORTED = 2, /* NotSupportedException: shape or dtype not built   */
    HYMT_E_CAPACITY = 3,    /* NotSupportedException: KV capacity exceeded       */
    HYMT_E_NO_DEVICE = 4,   /* PlatformNotSupportedException: no usable GPU      */
    HYMT_E_DEVICE = 5,      /* InvalidOperationException: a HIP call failed      */
    HYMT_E_OOM = 6,         /* OutOfMemoryException: device allocation failed    */
    HYMT_E_STATE = 7        /* InvalidOperationException: call out of order      */
} hymt_status;

/* KV cache / io element types. */
typedef enum hymt_dtype { HYMT_F32 = 0, HYMT_F16 = 1, HYMT_BF16 = 2 } hymt_dtype;

/* Tokens per KV page: the reference's Metal block size (MetalBackend.cs:49-50). */
#define HYMT_PAGE_TOKENS 64

/* hymt_create(device) value for a context with host bookkeeping only: the
 * page table works, every call that needs the GPU returns HYMT_E_NO_DEVICE. */
#define HYMT_DEVICE_NONE (-1)

/* Tensor pointers of this call are device pointers; the call is asynchronous. */
#define HYMT_FLAG_DEVICE_PTRS 1u

typedef struct hymt_ctx hymt_ctx;

/* Message of the last failing call on this thread ("" if none). */
const char *hymt_last_error(void);

/* HYMT_ABI_VERSION of the loaded library. */
int hymt_abi_version(void);

/* Number of HIP devices.  Replaces the device probe of BackendFactory's auto
 * mode (BackendFactory.cs:29-38, VulkanBackend.IsSupported). */
int hymt_device_count(int *count);

/* Open a context on `device` (or HYMT_DEVICE_NONE).  Replaces the backend
 * constructor (VulkanBackend.cs:80-89: throws when the device is unusable). */
int hymt_create(int device, hymt_ctx **out);

/* Free every device buffer of the context.  Replaces IDisposable.Dispose
 * (IComputeBackend.cs:14; the model disposes it, HunyuanDenseModel.cs:815-824). */
int hymt_destroy(hymt_ctx *ctx);

/* Attention hyper-parameters from ModelConfig (ModelConfig.cs:21-51): heads,
 * kv heads, head_dim, rope_dim, rope base (already alpha-scaled, :31-34) and
 * the RMSNorm eps (:49).  Built shapes: head_dim 128, heads/kv_heads = 4,
 * rope_dim even and <= head_dim.  Must precede hymt_kv_create. */
int hymt_set_attn_config(hymt_ctx *ctx, int heads, int kv_heads, int head_dim, int rope_dim,
                         float rope_base, float eps);

/* Allocate the paged K/V cache: `layers` layers, room for `max_tokens`
 * positions (rounded up to whole pages), elements of `kv_dtype`.  Replaces
 * the KV part of IComputeBackend.LoadModel (MetalBackend.cs:164-181). */
int hymt_kv_create(hymt_ctx *ctx, int layers, int max_tokens, int kv_dtype);

/* Capacity in tokens, pages in the pool, pages mapped by the page table. */
int hymt_kv_info(hymt_ctx *ctx, int *max_tokens, int *pages_total, int *pages_mapped);

/* Map pages for positions [pos, pos+len) ahead of writes (the reference's
 * EnsureWrittenRange, MetalBackend.cs:294-318).  Decode, prefill and upload
 * map what they write themselves; this is for callers that reserve early. */
int hymt_kv_map(hymt_ctx *ctx, int pos, int len);

/* Physical page of logical block `block` (-1 when unmapped): the host copy of
 * the page table (MetalBackend.cs:55 `_tab`). */
int hymt_kv_page(hymt_ctx *ctx, int block, int *phys);

/* Live cache length: blocks that start at or after `len` are unmapped and
 * their pages return to the free list unless the block store pins them.
 * Replaces IComputeBackend.SetCacheLen (IComputeBackend.cs:82-87). */
int hymt_kv_set_len(hymt_ctx *ctx, int len);

/*
 * Device block store (IComputeBackend.SupportsBlockStore = true,
 * DeviceBlockTokens = HYMT_PAGE_TOKENS; IComputeBackend.cs:49-87), after the
 * Metal backend's (MetalBackend.cs:224-387).  A full 64-token block of a
 * sequence is keyed by the chained FNV-1a hash of all tokens up to its end
 * (KvBlockStore.ChainHash, KvBlockStore.cs:51-60) and the key's tokens are
 * kept, so a hash collision is a miss.  Pinned pages are never written: a
 * later write into their block (decode, prefill, upload, hymt_kv_map) maps a
 * fresh page and first copies the pinned page into it in every layer when
 * the write starts inside the block.  When the pool runs out, entries are
 * evicted least recently harvested first, never while their page is mapped
 * in the live range.
 *
 * hymt_kv_harvest replaces HarvestPrefix: pins the page of every full block
 * of tokens[0, n_tokens) that is mapped.  hymt_kv_restore replaces
 * RestorePrefix: maps the longest run of full blocks of tokens[0, n_tokens)
 * found in the store, from block 0, and sets *restored_tokens to the number
 * of tokens restored (a multiple of 64); the caller then sets the cache
 * length (hymt_kv_set_len).  block_tokens other than 64 -> HYMT_E_UNSUPPORTED.
 * Neither may run while a recording is open.
 */
int hymt_kv_harvest(hymt_ctx *ctx, const int32_t *tokens, int n_tokens, int block_tokens);
int hymt_kv_restore(hymt_ctx *ctx, const int32_t *tokens, int n_tokens, int block_tokens,
                    int *restored_tokens);
/* Store entries and pages held by neither the table nor the store. */
int hymt_kv_store_info(hymt_ctx *ctx, int *entries, int *pages_free);

/* Copy rows [pos, pos+len) of one layer from the model's flat bf16 caches
 * (row j at k_bf16 + j*kv_stride) into the device cache, converting to the
 * cache dtype.  Replaces IComputeBackend.UploadKv (IComputeBackend.cs:31-38). */
int hymt_kv_upload(hymt_ctx *ctx, int layer, int pos, int len, const uint16_t *k_bf16,
                   const uint16_t *v_bf16);

/* Read rows [pos, pos+len) of one layer back as fp32 in the reference's row
 * layout (k_out[(j-pos)*kv_stride + kvh*head_dim + d]).  Host pointers.  The
 * debug dump of VulkanBackend.cs:909-1015 (HYMT_VK_DUMP) in a testable form. */
int hymt_kv_read(hymt_ctx *ctx, int layer, int pos, int len, float *k_out, float *v_out);

/*
 * Decode attention for one layer at position `pos` (1 token):
 * RoPE(q), RoPE(k) at pos -> RMSNorm q, k with qnw/knw -> append k, v at
 * row pos (rounded to the cache dtype) -> out = softmax(q K^T / sqrt(D)) V
 * over positions [0, pos], softmax floored at -80 as Ops.SoftmaxRow.
 * q [heads*D], k,v [kv_heads*D], qnw [D], knw [D], out [heads*D], fp32.
 * qnw/knw NULL skip that norm.  Rows [0, pos) must be resident.
 * Replaces HunyuanDenseModel.DecodeAttention lines 79-95
 * (HunyuanDenseModel.Decode.cs), i.e. the attention the Vulkan dec_attn2
 * kernel fuses (dec_attn2.comp:1-177).
 */
int hymt_attn_decode(hymt_ctx *ctx, int layer, int pos, const float *q, const float *k,
                     const float *v, const float *qnw, const float *knw, float *out,
                     unsigned flags);

/*
 * hymt_attn_decode for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It has no counterpart in the reference.  Device pointers only (as
 * HYMT_FLAG_DEVICE_PTRS), same arguments and result as hymt_attn_decode, and
 * it never calls hipMalloc or hipFree: the split partials live in a static
 * device array of the library (4.06 MiB per GPU, held until the process
 * ends; room for 32 q heads, a larger head count is HYMT_E_UNSUPPORTED), and
 * the RoPE table is built for the whole cache by hymt_kv_create.  One
 * context at a time owns a GPU's array: the first context to call this on a
 * GPU holds it until hymt_destroy, and a call from any other live context on
 * that GPU returns HYMT_E_STATE instead of racing on it.  The owner's calls
 * run in its stream's order; the array keeps the last call's partials.
 */
int hymt_attn_decode_noalloc(hymt_ctx *ctx, int layer, int pos, const float *q, const float *k,
                             const float *v, const float *qnw, const float *knw, float *out);

/*
 * Causal prefill attention for one layer: `seq` tokens at positions
 * [pos, pos+seq), attending over [0, pos+row].  Same steps as decode; K/V of
 * the chunk are written into the cache.  q/k/v are fp32 or bf16 as io_dtype;
 * out is fp32.  The row maximum starts at -80 as in Ops.SoftmaxRow; the
 * per-weight clamp at -80 below the maximum is not applied (such weights are
 * below 2e-35 of the largest, under fp32 resolution of the row sum).
 * Cache dtype f16 or bf16 (MFMA operand type); f32 caches
 * return HYMT_E_UNSUPPORTED.  The V rows after the chunk, up to the end of
 * the 64-position page that holds its last position, are set to zero (the
 * reference treats positions >= pos+seq as unwritten; ForwardStep's
 * postcondition covers [0, pos+seq) only, IComputeBackend.cs:40-47).
 * Replaces HunyuanDenseModel.PrefillAttention
 * lines 53-83 (HunyuanDenseModel.Prefill.cs), the pf_kvprep + pf_fa32 pair
 * of the Vulkan backend (VulkanBackend.cs:786-802).
 */
int hymt_attn_prefill(hymt_ctx *ctx, int layer, int pos, int seq, const void *q, const void *k,
                      const void *v, int io_dtype, const float *qnw, const float *knw, float *out,
                      unsigned flags);

/* hymt_attn_prefill over rows that are not packed: row j of q starts at
 * q + j*q_ld elements, of k and v at k + j*kv_ld and v + j*kv_ld (q_ld >=
 * heads*head_dim, kv_ld >= kv_heads*head_dim, both multiples of 8).  Lets
 * q, k and v be column ranges of one fused [seq][q|k|v] projection output,
 * as the Vulkan prefill reads its qkv buffer (pf_kvprep / pf_fa32 over
 * _pfQkv, VulkanBackend.cs:786-802).  Device pointers only. */
int hymt_attn_prefill_ld(hymt_ctx *ctx, int layer, int pos, int seq, const void *q, int q_ld, const void *k,
                         const void *v, int kv_ld, int io_dtype, const float *qnw, const float *knw,
                         float *out, unsigned flags);

/* Wait for all work on the context's stream. */
int hymt_sync(hymt_ctx *ctx);

/*
 * Per-kernel timing, the counterpart of the reference's HYMT_VK_TIMING and
 * HYMT_VK_PFPROF modes (VulkanBackend.cs:55,71-74,410-411,488-540).  Read from
 * the environment when a device context is created, and switched later with
 * hymt_timing_enable:
 *   HYMT_HIP_TIMING=1      every public call that enqueues kernels (attention,
 *                          GEMV/GEMM and row kernels, model step, replay)
 *                          records a HIP event pair around each kernel it
 *                          enqueues, waits for them when it ends and prints
 *                          one line to stderr, "[hymt timing] <call>(<arg>):
 *                          <us> us on the GPU, <n> kernels | <kernel> <count>x
 *                          <us> us | ..."; hymt_destroy prints the totals;
 *   HYMT_HIP_TIMING=quiet  the same totals without printing.
 * Timed calls wait for their own kernels; calls being recorded are not timed.
 * hymt_timing_get returns one kernel's totals (count, summed microseconds)
 * over the calls timed since creation or hymt_timing_reset; HYMT_E_STATE when
 * the context does not time, HYMT_E_ARG for a kernel never timed.  Kernel
 * names: decode_attn, decode_merge, prefill_kv, prefill_flash, prefill_merge,
 * gemv_<type>, gemm_bf16_out_{f32,bf16}, rows_*, kv_*, embed, weight_rows,
 * tab_update, graph (a whole replay).
 */
/* mode 0 stops timing (the totals are kept), 1 times and prints, 2 times
 * quietly; a device context only (HYMT_E_NO_DEVICE otherwise). */
int hymt_timing_enable(hymt_ctx *ctx, int mode);
int hymt_timing_get(hymt_ctx *ctx, const char *kernel, long *count, double *us);
int hymt_timing_reset(hymt_ctx *ctx);

/*
 * Recorded call sequences (HIP graphs).  Between hymt_graph_begin and
 * hymt_graph_end the context's stream is captured: device-pointer
 * (HYMT_FLAG_DEVICE_PTRS) attention calls are recorded instead of run, and
 * hymt_graph_launch replays the whole sequence with one submission.  This is
 * the HIP form of the reference's recorded decode command buffer: the Vulkan
 * backend records the decode graph once (VulkanBackend.cs:326, RecordDecodeGraph
 * :400-568) and submits it per token (:677).  Replays repeat the recorded
 * arguments (positions included).  During capture, calls that synchronise,
 * copy host memory or would grow a device workspace return HYMT_E_STATE, so a
 * sequence is warmed up once eagerly before it is recorded.  A recording
 * holds the addresses of the context's workspaces: when a later eager call
 * grows one of them, hymt_graph_launch refuses the recording (HYMT_E_STATE)
 * and it must be recorded again.  Such a refusal
 * spoils the recording: it stays open, and hymt_graph_end discards it and
 * reports the failure.  A call rejected for its arguments records nothing
 * and leaves the recording intact.
 */
typedef struct hymt_graph hymt_graph;
int hymt_graph_begin(hymt_ctx *ctx);
int hymt_graph_end(hymt_ctx *ctx, hymt_graph **graph);
int hymt_graph_launch(hymt_ctx *ctx, hymt_graph *graph);
int hymt_graph_destroy(hymt_ctx *ctx, hymt_graph *graph);

/* The context's hipStream_t, for callers that time or order work around it. */
int hymt_get_stream(hymt_ctx *ctx, void **stream);

/* Device buffers for callers that keep activations resident
 * (HYMT_FLAG_DEVICE_PTRS) and host<->device copies on the context's stream.
 * kind: 0 host->device, 1 device->host, 2 device->device.  Copies wait for
 * completion before returning. */
int hymt_dev_alloc(hymt_ctx *ctx, size_t bytes, void **dptr);
int hymt_dev_free(hymt_ctx *ctx, void *dptr);
int hymt_memcpy(hymt_ctx *ctx, void *dst, const void *src, size_t bytes, int kind);

/* ---- quantized weights and the decode GEMV ------------------------------------
 * The weight half of IComputeBackend.LoadModel (IComputeBackend.cs:25-29) and of
 * the decode graph's matrix-vector products (HunyuanDenseModel.Decode.cs
 * DecodeQkv / DecodeLinear / DecodeGateUp; VulkanBackend.cs:400-568 with
 * dec_gemvadd_*.comp): a matrix of rows x cols values arrives as the rows of
 * GGUF blocks GgufFile hands the reference's kernels (GgufFile.cs:111), in one
 * of the types below (GgmlTensorType.cs codes), and is repacked into the
 * device layout.  cols must be a multiple of 2048 up to 8192 (the model's
 * 2048 and 6144). */
#define HYMT_W_F32 0
#define HYMT_W_F16 1
#define HYMT_W_Q8_0 8
#define HYMT_W_Q4_K 12
#define HYMT_W_Q6_K 14
#define HYMT_W_Q2_0C 40
#define HYMT_W_STQ1_0 43

typedef struct hymt_weight hymt_weight;

/* Upload (host data, `bytes` = rows x the type's row bytes).  Not recordable. */
int hymt_weight_upload(hymt_ctx *ctx, int type, int rows, int cols, const void *data, size_t bytes,
                       hymt_weight **out);
int hymt_weight_free(hymt_ctx *ctx, hymt_weight *w);
int hymt_weight_info(const hymt_weight *w, int *type, int *rows, int *cols, size_t *device_bytes);

/* y[rows] = W x'[cols], or y += W x' with HYMT_GEMV_ACCUMULATE (the residual
 * add of dec_gemvadd_*), where x' is x as the input flags make it:
 *   HYMT_GEMV_IN_RMSNORM  x' = x / sqrt(mean(x^2) + eps) * norm_w[cols]
 *                         (Ops.RmsNorm, Ops.cs:12-90: the RMSNorm before a
 *                         block's projections, dec_prekv / dec_preffn)
 *   HYMT_GEMV_IN_SWIGLU   x holds gate[cols] then up[cols];
 *                         x' = gate / (1 + exp(-gate)) * up (Ops.SiLUMul,
 *                         Ops.cs:999-1052: the FFN's down projection input)
 * and the output as HYMT_GEMV_OUT_SWIGLU makes it:
 *   HYMT_GEMV_OUT_SWIGLU  W is [gate; up] (rows = 2 F); y[F] = silu(gate) * up
 *                         with gate = W[0:F] x', up = W[F:2F] x' (the fused
 *                         gate/up of the reference's Vulkan decode,
 *                         dec_ffngu.comp:9-11, 292-301; excludes ACCUMULATE)
 * x, y and norm_w are device pointers (x and norm_w 16-byte aligned); the call
 * only enqueues work and may be recorded.  fp32 activations and accumulation. */
#define HYMT_GEMV_ACCUMULATE 1
#define HYMT_GEMV_IN_RMSNORM 2
#define HYMT_GEMV_IN_SWIGLU 4
#define HYMT_GEMV_OUT_SWIGLU 8
int hymt_gemv(hymt_ctx *ctx, const hymt_weight *w, const float *x, float *y, int flags,
              const float *norm_w, float eps);

/* out[cols] = row `row` of W, dequantized (the embedding lookup,
 * HunyuanDenseModel.Embed, HunyuanDenseModel.cs:494-557).  out is a device
 * pointer; the call only enqueues work and may be recorded. */
int hymt_embed(hymt_ctx *ctx, const hymt_weight *w, int row, float *out);

/* ---- prefill: dense weights, GEMMs and row kernels ----------------------------
 * The prefill half of ForwardStep (HunyuanDenseModel.Forward's prefill blocks,
 * HunyuanDenseModel.Prefill.cs; the Vulkan prefill sequence of
 * VulkanBackend.cs:760-880, which keeps 16-bit dense copies of the layer
 * weights and runs GEMMs over the prompt's rows).  Matrices are row-major;
 * bf16 values are uint16 bit patterns rounded to nearest even. */

/* Give the weight a bf16 [rows][cols] dense copy of its dequantized values
 * (held until hymt_weight_free; 2 bytes per value of device memory).
 * Synchronous; not recordable. */
int hymt_weight_dense(hymt_ctx *ctx, hymt_weight *w);

/* y[m][nrows] = x[m][cols] . W[row0 : row0+nrows][cols]^T over the dense
 * copy, bf16 operands and fp32 accumulation (the Gemm calls of
 * VulkanBackend.cs:782-856).  y is fp32 [m][nrows], bf16 with
 * HYMT_GEMM_OUT_BF16, or fp32 accumulated into (y +=, the residual add) with
 * HYMT_GEMM_ACCUMULATE.  x, y device pointers; not recordable. */
#define HYMT_GEMM_ACCUMULATE 1
#define HYMT_GEMM_OUT_BF16 2
int hymt_gemm(hymt_ctx *ctx, const hymt_weight *w, int row0, int nrows, const void *x, int m, void *y,
              int flags);

/* out[i][cols] = row rows[i] of W dequantized, fp32 (the prompt's embedding,
 * HunyuanDenseModel.Embed, HunyuanDenseModel.cs:494-557).  rows is a host
 * array, out a device pointer; returns when the rows are written. */
int hymt_embed_rows(hymt_ctx *ctx, const hymt_weight *w, const int32_t *rows, int n, float *out);

/* out[i] = bf16(x[i] / sqrt(mean(x[i]^2) + eps) * norm_w) for m rows of n
 * fp32 values (Ops.RmsNorm, Ops.cs:12-90).  n a multiple of 4 up to 8192.
 * For this and the two calls below: fp32 inputs 16-byte aligned, bf16
 * outputs 8-byte aligned (vector loads and stores). */
int hymt_rows_rmsnorm(hymt_ctx *ctx, const float *x, int m, int n, const float *norm_w, float eps, void *out);

/* out[i][j] = bf16(g / (1 + exp(-g)) * u), g = gate_up[i][j], u =
 * gate_up[i][n + j] (Ops.SiLUMul, Ops.cs:999-1052). */
int hymt_rows_swiglu(hymt_ctx *ctx, const float *gate_up, int m, int n, void *out);

/* hymt_rows_swiglu over a bf16 gate_up (a HYMT_GEMM_OUT_BF16 GEMM output);
 * gate_up and out 8-byte aligned. */
int hymt_rows_swiglu_bf16(hymt_ctx *ctx, const void *gate_up, int m, int n, void *out);

/* out[i] = bf16(x[i]) for count fp32 values (count a multiple of 4). */
int hymt_to_bf16(hymt_ctx *ctx, const float *x, size_t count, void *out);

/* act[m][f] = bf16(silu(g) u), g and u the bf16 products x . Wg^T and
 * x . Wu^T over the dense copies: the gate/up GEMM with SwiGLU fused into
 * its output, one launch (the reference's Gemm(..., swiglu: true), and the
 * Gemm + pf_silumul pair it replaces, VulkanBackend.cs:845-853).  gate is
 * one weight of 2 f rows [gate; up] with up NULL, or the f gate rows with up
 * the f up rows.  It runs only where its bits equal those of hymt_gemm with
 * HYMT_GEMM_OUT_BF16 into a bf16 [m][2 f] buffer (the two halves by two calls
 * for two weights) followed by hymt_rows_swiglu_bf16: the context's GEMM
 * choice is the hand-written MFMA kernel, unsplit, for those calls, f a
 * multiple of 64, cols a multiple of 128; otherwise it returns
 * HYMT_E_UNSUPPORTED and enqueues nothing, and the caller issues those calls.
 * x, act device pointers, 16-byte aligned; not recordable. */
int hymt_gemm_swiglu(hymt_ctx *ctx, const hymt_weight *gate, const hymt_weight *up, const void *x, int m,
                     void *act);

/* ---- the model's decode step, enqueued natively ---------------------------------
 * IComputeBackend.ForwardStep for one token (IComputeBackend.cs:40-47) in one
 * call: the sequence of HunyuanDenseModel.DecodeBlock
 * (HunyuanDenseModel.Decode.cs:30-101) over weights already uploaded --
 *   h = token_embd[token]
 *   per layer: qkv = W_qkv RMSNorm(h, attn_norm); ao = decode attention at pos
 *              (RoPE, QK norm, append); h += W_o ao;
 *              gu = W_gate|up RMSNorm(h, ffn_norm); h += W_down (silu(gate) * up)
 *   logits = W_out RMSNorm(h, output_norm)
 * -- i.e. hymt_embed, hymt_gemv and hymt_attn_decode with device pointers, on the
 * context's stream (recordable).  The model borrows the weights and norm
 * vectors (device pointers, 16-byte aligned) and owns its activation
 * buffers; destroy it before its weights and the context.  The context's KV
 * cache must have `layers` layers. */
typedef struct hymt_model hymt_model;
int hymt_model_create(hymt_ctx *ctx, int layers, int hidden, int ffn, int vocab, float eps, hymt_model **model);
/* q_or_qkv: [q; k; v] rows (k = v = NULL) or q alone with k and v;
 * gate_or_gate_up: [gate; up] rows (up = NULL) or gate alone with up.
 * q_norm / k_norm may be NULL (no QK norm). */
int hymt_model_set_layer(hymt_model *model, int layer, const hymt_weight *q_or_qkv, const hymt_weight *k,
                         const hymt_weight *v, const hymt_weight *o, const hymt_weight *gate_or_gate_up,
                         const hymt_weight *up, const hymt_weight *down, const float *attn_norm,
                         const float *ffn_norm, const float *q_norm, const float *k_norm);
/* out NULL: the output projection uses the tied embedding (HunyuanDenseModel.cs:419). */
int hymt_model_set_io(hymt_model *model, const hymt_weight *token_embd, const hymt_weight *out,
                      const float *out_norm);
/* Enqueue the decode step of `token` at `pos`; logits: device pointer, vocab floats. */
int hymt_model_decode(hymt_model *model, int token, int pos, float *logits);

/* IComputeBackend.ForwardStep for n >= 1 tokens at positions [pos, pos+n)
 * (IComputeBackend.cs:40-47) in one call: the prompt runs as prefill chunks
 * of up to 2048 rows (Forward chunks by 1024, HunyuanDenseModel.cs:342-355;
 * the result does not depend on the chunking), the Vulkan backend's recorded
 * prefill (VulkanBackend.cs:760-880, 1017-1062) as native calls --
 *   X = token_embd[tokens]
 *   per layer: XN = bf16 RMSNorm(X, attn_norm); [Q|K|V] = XN W_qkv^T (bf16)
 *              AO = causal prefill attention (RoPE, QK norm, append)
 *              X += bf16(AO) W_o^T
 *              GU = bf16 RMSNorm(X, ffn_norm) W_gate|up^T
 *              X += bf16(silu(gate) * up) W_down^T
 *   logits = W_out RMSNorm(X[n-1], output_norm)
 * -- over the layer weights' bf16 dense copies (hymt_weight_dense), bf16 GEMM
 * operands with fp32 accumulation.  GU is bf16 unless
 * HYMT_PREFILL_GATE_UP_F32 keeps it fp32 as the reference's prefill does
 * (its _pfGu buffer, VulkanBackend.cs:595,604); bf16 GU adds two bf16
 * roundings per FFN element.  With n = 1, an fp32 cache, or a layer weight
 * without a dense copy, the tokens run as decode steps (hymt_model_decode).
 * tokens is a host array (read before the call returns); logits a device
 * pointer (vocab floats, the last token's).  Not recordable. */
#define HYMT_PREFILL_GATE_UP_F32 1u
int hymt_model_prefill(hymt_model *model, const int32_t *tokens, int n, int pos, float *logits,
                       unsigned flags);
int hymt_model_destroy(hymt_model *model);

#ifdef __cplusplus
}
#endif

#endif
