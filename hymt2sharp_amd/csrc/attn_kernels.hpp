// attn_kernels.hpp -- argument blocks and host launchers of the gfx950
// attention kernels.  Included by the C-ABI shim (hymt_hip.cpp) and by the
// kernel sources.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hymt {

constexpr int kHeadDim = 128;   // built head_dim (Hy-MT2-1.8B)
constexpr int kGroup = 4;       // q heads per kv head (16 / 4)
constexpr int kPage = 64;       // tokens per KV page
constexpr int kMaxSplits = 256; // decode KV splits per kv head (merge width)
constexpr int kArgPages = 256;  // decode page lists passed in kernel arguments
constexpr int kItemTiles = 1024; // prefill kv tiles per work item (page ids staged in LDS)

// Paged pool addressing, per layer.  A page holds 64 positions of one kv head
// for K and for V; page_base = (phys*Hkv + kvh) * 64 * D elements.
//
// f16/bf16 pages (16 KiB each) hold 16-byte chunks of 8 elements in MFMA
// operand order, so that the operand loads of every kernel, and the copies
// that stage a page into LDS, are linear 1 KiB wave accesses:
//   K  chunk (s, j, c) = dims 8j..8j+7 of position 16s + c, at chunk index
//      (16 s + j) * 16 + c.  Sub-tile s (16 positions) is one 4 KiB block;
//      16 lanes reading dim chunk j of its 16 positions read 256 bytes.
//   V  chunk (pc, d) = 8 positions of dim d, at chunk index pc * D + d.
//      Chunk pc = 4m + g holds positions 32m + 4g + [0, 4) followed by
//      32m + 16 + 4g + [0, 4): lane (g, c) of a 16x16 S^T MFMA output holds
//      rows 4g + [0, 4), so the outputs of the two 16-position blocks of one
//      32-position step form the P.V operand that meets this chunk.
// f32 pages (VALU decode only): K row-major t*D + d; V transposed in
// 16-position sub-tiles ((t/16)*D + d)*16 + t%16.
__host__ __device__ inline size_t k_off16(int t, int d) {
    return ((size_t)(((t >> 4) * 16 + (d >> 3)) * 16 + (t & 15)) << 3) + (d & 7);
}
// position of element e of V chunk pc (f16/bf16 pages)
__host__ __device__ inline int v_chunk_pos(int pc, int e) {
    return 32 * (pc >> 2) + 4 * (pc & 3) + 16 * (e >> 2) + (e & 3);
}
__host__ __device__ inline size_t v_off16(int t, int d) {
    const int pc = 4 * (t >> 5) + ((t >> 2) & 3), e = 4 * ((t >> 4) & 1) + (t & 3);
    return ((size_t)pc * kHeadDim + d) * 8 + e;
}
__host__ __device__ inline size_t k_off32(int t, int d) { return (size_t)t * kHeadDim + d; }
__host__ __device__ inline size_t v_off32(int t, int d) {
    return ((size_t)(t >> 4) * kHeadDim + d) * 16 + (t & 15);
}
// by element size: 4 -> f32 page, 2 -> f16/bf16 page
template <int BYTES> __host__ __device__ inline size_t k_off(int t, int d) {
    return BYTES == 4 ? k_off32(t, d) : k_off16(t, d);
}
template <int BYTES> __host__ __device__ inline size_t v_off(int t, int d) {
    return BYTES == 4 ? v_off32(t, d) : v_off16(t, d);
}

struct DecodeArgs {
    // Ordered for the kernel's prologue, which is one batch of scalar
    // argument loads: the page ids (the K/V addresses hang on them), then the
    // pointers and scalars of the first vector loads.  Every pointer is
    // valid: an absent gamma or RoPE table is a ones vector.
    int32_t pages[kArgPages];  // physical page of each logical block (when
                               // pages_in_args), saving a dependent table load
    const void *kpool;      // this layer's K pool
    const void *vpool;      // this layer's V pool
    const float *q;         // [Hq*D]
    const float *knew;      // [Hkv*D]
    const float *vnew;      // [Hkv*D]
    const float *qnw;       // [D] gamma of q
    const float *knw;       // [D] gamma of k
    const float *rope_cos;  // row `pos` of the cos table, [rope_half]
    const float *rope_sin;
    int L;                  // positions attended = pos + 1
    int kv_heads;
    int ppw;                // pages per split (set by launch_decode)
    int nsplit;             // splits per kv head (set by launch_decode)
    int rope_half;
    int rope_dim;
    int norm_q, norm_k;     // apply the q / k RMSNorm
    float eps;
    float qscale;           // log2(e) / sqrt(D)
    int pages_in_args;      // 1: pages[] holds tab[0, ceil(L/64)) (<= kArgPages)
    const int32_t *tab;     // logical block -> physical page
    float *out;             // [Hq*D]
    float *part_ml;         // [Hq][kMaxSplits][2]
    float *part_acc;        // [Hq][kMaxSplits][D]
};

struct PrepArgs {
    const void *k;      // [seq][Hkv*D]   fp32 or bf16 (io_bf16)
    const void *v;
    const float *knw;   // [D] gamma of k (a ones vector when the norm is off)
    const float *rope_cos; // table base [cap][rope_half]
    const float *rope_sin;
    const int32_t *tab;
    void *kpool, *vpool;
    int pos0, seq;
    int kv_heads;
    int rope_half, rope_dim;
    int io_bf16;
    int norm_k;         // apply the k RMSNorm
    float eps;
    int kv_ld;          // elements from one k (and v) row to the next, >= Hkv*D
    // with qready (split flash items): q prepared for prefill_flash in the
    // same launch (grid rows kv_heads and up), RoPE + RMSNorm + the softmax
    // scale, rounded to the cache type
    const void *q;      // [seq][q_ld]    fp32 or bf16 (io_bf16)
    const float *qnw;   // [D] gamma of q (a ones vector when the norm is off)
    void *qready;       // [seq][heads*D] in the cache type, or null
    int q_ld, heads, norm_q;
    float qscale;       // log2(e) / sqrt(D)
};

struct FlashArgs {
    const void *q;      // [seq][Hq*D]    fp32 or bf16 (io_bf16), before RoPE/norm
    const float *qnw;   // [D] gamma of q (a ones vector when the norm is off)
    const uint16_t *qready;  // null, or [seq][Hq*D] q after RoPE, norm and qscale in the cache type (prefill_kv)
    const float *rope_cos, *rope_sin;  // table base [cap][rope_half]
    const int32_t *tab;
    const void *kpool, *vpool;
    float *out;         // [seq][Hq*D], fp32, or bf16 bits (RNE) when out_bf16
    void *part_o;       // [Hkv*items][G][32][D] O / l in the cache type (split items only)
    float *part_ml;     // [Hkv*items][G][32][2] (m, l)
    int pos0, seq;
    int heads, kv_heads;
    int rope_half, rope_dim;  // rope_dim in {0, 64, 128}
    int io_bf16;
    int norm_q;         // apply the q RMSNorm
    float eps, qscale;  // qscale = log2(e) / sqrt(D)
    int nb16;           // q blocks of 16 rows
    int npairs;         // block pairs (b, nb16-1-b), b < npairs
    int cap;            // max kv tiles per work item
    int items_per_kvh;  // work items per kv head
    int q_ld;           // elements from one q row to the next, >= Hq*D
    int out_bf16;       // write out as bf16 (the input of a bf16 GEMM)
    int split_ns;       // > 1: every pair splits into this many items (item = pair * split_ns + split)
    int pages_in_args;  // 1: pages[] holds tab[0, ceil((pos0+seq)/64)) (<= kArgPages)
    int32_t pages[kArgPages];  // physical page of each logical block (when
                               // pages_in_args): the first tile's copy then
                               // waits for no table load
};

// Number of kv tiles (pages) the 16-row q block b attends to.
__host__ __device__ inline int block_tiles(int pos0, int b, int seq) {
    int last = pos0 + b * 16 + 15;
    int lim = pos0 + seq - 1;
    if (last > lim) last = lim;
    return last / 64 + 1;
}

// Causal prefill pairs the short block b with the long block nb16-1-b, so
// every pair carries about the same work.  The long block sets the pair's
// kv range; the short one (absent for the middle block of an odd count)
// joins for the tiles it attends to.
__host__ __device__ inline int pair_tiles(int pos0, int pair, int nb16, int seq) {
    return block_tiles(pos0, nb16 - 1 - pair, seq);
}

// kv dtype codes as in hymt_dtype.
hipError_t launch_decode(int kv_dtype, const DecodeArgs &a, hipStream_t s);
// The static decode workspace (decode_attn.hip): resolve its address on
// `device` (call with that device current, once per device), then fetch it.
hipError_t decode_scratch_init(int device);
hipError_t decode_scratch(int device, float **part_ml, float **part_acc, int *max_heads);
// Ownership of a device's static decode workspace: claim succeeds for the
// owner or when the device has none; release clears it (owner only).
bool decode_scratch_claim(int device, const void *owner);
void decode_scratch_release(int device, const void *owner);
hipError_t launch_prefill_prep(int kv_dtype, const PrepArgs &a, hipStream_t s);
hipError_t launch_prefill_flash(int kv_dtype, const FlashArgs &a, int total_items, hipStream_t s);
hipError_t launch_prefill_merge(int kv_dtype, const FlashArgs &a, hipStream_t s);
hipError_t launch_tab_update(int32_t *tab, const int *idx, const int *val, int n, hipStream_t s);
hipError_t launch_kv_copy_page(void *kpool, void *vpool, size_t layer_bytes, size_t page_bytes, int src,
                               int dst, int layers, hipStream_t s);
hipError_t launch_kv_upload(int kv_dtype, const uint16_t *k_bf16, const uint16_t *v_bf16,
                            const int32_t *tab, void *kpool, void *vpool, int pos, int len,
                            int kv_heads, hipStream_t s);
hipError_t launch_kv_read(int kv_dtype, const int32_t *tab, const void *kpool, const void *vpool,
                          float *k_out, float *v_out, int pos, int len, int kv_heads,
                          hipStream_t s);

}  // namespace hymt
