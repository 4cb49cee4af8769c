// prefill_attn.hip -- causal GQA prefill attention for gfx950.
//
// Replaces the prefill attention of HunyuanDenseModel.PrefillAttention
// (HunyuanDenseModel.Prefill.cs:53-83): RoPE + Q/K RMSNorm + append of the
// chunk's K/V, then AttentionScores -> SoftmaxCausal -> AttentionCombine
// (Ops.cs:198-221, 359-455, 535-595), as the Vulkan pf_kvprep + pf_fa32 pair
// does on other GPUs (pf_kvprep.comp, pf_fa32.comp).
//
// Kernels:
//  prefill_kv     one workgroup per (32-position block, kv head): RoPE + norm
//                 of k, k and v rounded into the paged cache (v transposed
//                 through LDS into whole V chunks); when the flash items are
//                 split, also one per (32-position block, q head): RoPE +
//                 norm of the q rows times the softmax scale, rounded to the
//                 operand type (qready), which the split items then load
//                 instead of each preparing the same rows again.
//  prefill_flash  one workgroup per (kv head, 32-row q block, kv tile range):
//                 8 waves = the 4 q heads of the GQA group x the two parities
//                 of the range's 64-position tiles, so every SIMD runs two
//                 waves; each staged K/V tile in LDS serves the 4 heads.  The
//                 prologue applies RoPE + norm to the wave's 32 q rows
//                 straight into MFMA operand registers (or, QREADY, loads
//                 them prepared by prefill_kv).  S^T - m = K Q^T - m
//                 (accumulated onto -m) and O^T += V^T P^T on
//                 v_mfma_f32_16x16x32_{bf16,f16}; single-pass online softmax
//                 in base 2 with a lazy running maximum that starts at the
//                 reference's -80; the two parities merge through LDS.
//                 The reference clamps each exponent at -80 below the row
//                 maximum; weights that small (< 2e-35 of the largest) are
//                 below fp32 resolution of the row sum, so the kernel uses
//                 the exact exponent.
//  prefill_merge  combines the (m, l, O) partials of q blocks whose kv range
//                 was split over several workgroups (long cached prefixes).
#include <type_traits>

#include "attn_kernels.hpp"
#include "device_common.hpp"
#include "ktimer.hpp"

namespace hymt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Cross-row (16-lane) reductions with the gfx950 permlane swaps.
__device__ __forceinline__ float pf_xrow_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pf_xrow_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Two floats to the MFMA operand type, packed (v_cvt_pk_{bf16,f16}_f32, RNE).
template <typename T> __device__ __forceinline__ uint32_t pack2(float x, float y);
template <> __device__ __forceinline__ uint32_t pack2<BF16>(float x, float y) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    v2 r;
    r[0] = (__bf16)x;
    r[1] = (__bf16)y;
    return __builtin_bit_cast(uint32_t, r);
}
template <> __device__ __forceinline__ uint32_t pack2<F16>(float x, float y) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    v2 r;
    r[0] = (_Float16)x;
    r[1] = (_Float16)y;
    return __builtin_bit_cast(uint32_t, r);
}

// Load 8 consecutive input elements (fp32 or bf16 bits) as fp32.
__device__ __forceinline__ void load8_in(const void *base, size_t i, bool bf16, float *o) {
    if (bf16) {
        const uint4 u = *(const uint4 *)((const uint16_t *)base + i);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            o[2 * e] = __uint_as_float(w[e] << 16);
            o[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
        }
    } else {
        const float4 a = *(const float4 *)((const float *)base + i);
        const float4 b = *(const float4 *)((const float *)base + i + 4);
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
}

// ------------------------------------------------------------------ k/v
// Block (32-position block, kv head); thread (row = tid/16, dims 8*(tid%16)..).
// Straight-line loads, no branch between them (a load under a branch is
// followed by a wait before the next one): the row's page id first (only
// the stores need it), then k, v, the row's cos/sin and gamma (the host
// passes a ones vector when the norm is off).  The RoPE partner of dim d
// (d +- rope_dim/2) lives in lane c ^ (rope_dim/16) of the same 16-lane row
// and is fetched by DPP; the norm's sum of squares is a DPP reduction over
// the row.  K is written as one 16-byte store per thread.  V is transposed
// through LDS: a V chunk holds 8 positions of one 32-position step, so a
// block of 32 writes every chunk whole, 1 KiB per wave in one run (blocks
// of 16 would each write half of every chunk, 8 bytes at a time, and two
// workgroups on different XCDs would share each cache line).
// IN_BF16: k/v rows are bf16 (else fp32); HK = rope_dim / 64 in {0, 1, 2}.
template <int HK> __device__ __forceinline__ float rope_partner_dpp(float x, int c) {
    if constexpr (HK == 2) {  // c ^ 8: rotate the 16-lane row by 8
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
    } else {  // c ^ 4: from c + 4 (row_shl:4) or from c - 4 (row_shr:4)
        const float up = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x104, 0xF, 0xF, false));
        const float dn = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xF, 0xF, false));
        return (c & 4) ? dn : up;
    }
}

// q row m of head h for the split flash items: lane c of the row's 16 takes
// dims 8 c .. 8 c + 7 -- RoPE (partner by DPP, as for k below), RMSNorm (sum
// of squares by DPP over the row), gamma, the softmax scale log2(e)/sqrt(D),
// rounded to the cache type -- one 16-byte load and one 16-byte store.
template <typename T, bool IN_BF16, int HK>
__device__ __forceinline__ void q_row(const PrepArgs &a, int h, int m, int mc, bool valid, int c) {
    constexpr int D = kHeadDim;
    const int d0 = 8 * c, rh = a.rope_half;
    const size_t src = (size_t)mc * a.q_ld + (size_t)h * D + d0;
    float x[8], cs[8], sn[8], gw[8];
    if constexpr (IN_BF16) {
        const uint4 u = *(const uint4 *)((const uint16_t *)a.q + src);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[2 * e] = __uint_as_float(w[e] << 16);
            x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
        }
    } else {
        const float4 q0 = *(const float4 *)((const float *)a.q + src), q1 = *(const float4 *)((const float *)a.q + src + 4);
        x[0] = q0.x; x[1] = q0.y; x[2] = q0.z; x[3] = q0.w; x[4] = q1.x; x[5] = q1.y; x[6] = q1.z; x[7] = q1.w;
    }
    if constexpr (HK > 0) {
        const size_t rb = (size_t)(a.pos0 + mc) * rh + (d0 & (rh - 1));
        const float4 c0 = *(const float4 *)(a.rope_cos + rb), c1 = *(const float4 *)(a.rope_cos + rb + 4);
        const float4 s0 = *(const float4 *)(a.rope_sin + rb), s1 = *(const float4 *)(a.rope_sin + rb + 4);
        cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w; cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
        sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
    }
    {
        const float4 g0 = *(const float4 *)(a.qnw + d0), g1 = *(const float4 *)(a.qnw + d0 + 4);
        gw[0] = g0.x; gw[1] = g0.y; gw[2] = g0.z; gw[3] = g0.w; gw[4] = g1.x; gw[5] = g1.y; gw[6] = g1.z; gw[7] = g1.w;
    }
    float y[8], ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float yv = x[e];
        if constexpr (HK > 0) {
            const float xp = rope_partner_dpp<HK>(x[e], c);
            const bool rot = d0 < 64 * HK, lower = (d0 & rh) == 0;
            yv = !rot ? x[e] : lower ? x[e] * cs[e] - xp * sn[e] : xp * sn[e] + x[e] * cs[e];
        }
        y[e] = yv;
        ss += yv * yv;
    }
    ss = dpp_sum16(ss);
    const float rr = a.norm_q ? 1.0f / sqrtf(ss / (float)D + a.eps) : 1.0f;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        w[e] = (uint32_t)to_elem<T>(y[2 * e] * rr * gw[2 * e] * a.qscale) |
               ((uint32_t)to_elem<T>(y[2 * e + 1] * rr * gw[2 * e + 1] * a.qscale) << 16);
    if (valid)
        *(uint4 *)((uint16_t *)a.qready + (size_t)m * a.heads * D + (size_t)h * D + d0) = make_uint4(w[0], w[1], w[2], w[3]);
}

template <typename T, bool IN_BF16, int HK>
__global__ __launch_bounds__(512) void prefill_kv_kernel(PrepArgs a) {
    constexpr int D = kHeadDim, P = kPage;
    using S = typename T::storage;
    static_assert(sizeof(S) == 2, "prefill caches are 16-bit");
    __shared__ __attribute__((aligned(16))) S s_v[32][D];
    const int kvh = blockIdx.y, Hkv = a.kv_heads;
    const int tid = threadIdx.x, r = tid >> 4, c = tid & 15;
    const int pstart = (a.pos0 & ~31) + 32 * blockIdx.x;  // 32-aligned block start
    const int m = pstart + r - a.pos0;                    // row within the chunk
    const bool valid = m >= 0 && m < a.seq;
    const int mc = m < 0 ? 0 : (m < a.seq ? m : a.seq - 1);  // clamped for loads
    if (kvh >= Hkv) {  // a q block: head kvh - Hkv (uniform over the workgroup)
        q_row<T, IN_BF16, HK>(a, kvh - Hkv, m, mc, valid, c);
        return;
    }
    const int phys = __builtin_amdgcn_readfirstlane(a.tab[pstart / P]);
    const int d0 = 8 * c, rh = a.rope_half;
    const size_t src = (size_t)mc * a.kv_ld + (size_t)kvh * D + d0;

    float x[8], v[8], cs[8], sn[8], gw[8];
    if constexpr (IN_BF16) {
        const uint4 ku = *(const uint4 *)((const uint16_t *)a.k + src);
        const uint4 vu = *(const uint4 *)((const uint16_t *)a.v + src);
        const uint32_t kw[4] = {ku.x, ku.y, ku.z, ku.w}, vw[4] = {vu.x, vu.y, vu.z, vu.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[2 * e] = __uint_as_float(kw[e] << 16);
            x[2 * e + 1] = __uint_as_float(kw[e] & 0xFFFF0000u);
            v[2 * e] = __uint_as_float(vw[e] << 16);
            v[2 * e + 1] = __uint_as_float(vw[e] & 0xFFFF0000u);
        }
    } else {
        const float4 k0 = *(const float4 *)((const float *)a.k + src), k1 = *(const float4 *)((const float *)a.k + src + 4);
        const float4 v0 = *(const float4 *)((const float *)a.v + src), v1 = *(const float4 *)((const float *)a.v + src + 4);
        x[0] = k0.x; x[1] = k0.y; x[2] = k0.z; x[3] = k0.w; x[4] = k1.x; x[5] = k1.y; x[6] = k1.z; x[7] = k1.w;
        v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w; v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
    }
    if constexpr (HK > 0) {
        // every lane loads a table row (non-rotated dims of rope_dim 64 read
        // the row of dim d0 % 32 and ignore it)
        const size_t rb = (size_t)(a.pos0 + mc) * rh + (d0 & (rh - 1));
        const float4 c0 = *(const float4 *)(a.rope_cos + rb), c1 = *(const float4 *)(a.rope_cos + rb + 4);
        const float4 s0 = *(const float4 *)(a.rope_sin + rb), s1 = *(const float4 *)(a.rope_sin + rb + 4);
        cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w; cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
        sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
    }
    {
        const float4 g0 = *(const float4 *)(a.knw + d0), g1 = *(const float4 *)(a.knw + d0 + 4);
        gw[0] = g0.x; gw[1] = g0.y; gw[2] = g0.z; gw[3] = g0.w; gw[4] = g1.x; gw[5] = g1.y; gw[6] = g1.z; gw[7] = g1.w;
    }

    // V: round into LDS now, transpose after the barrier below.  Rows past
    // the chunk (up to the end of its last page) are stored as zeros: the
    // flash kernel stages whole pages, and P = 0 there must not meet NaN bits.
    {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            w[e] = (uint32_t)to_elem<T>(v[2 * e]) | ((uint32_t)to_elem<T>(v[2 * e + 1]) << 16);
        *(uint4 *)&s_v[r][d0] = m < a.seq ? make_uint4(w[0], w[1], w[2], w[3]) : make_uint4(0, 0, 0, 0);
    }

    // RoPE (Ops.RopeRange, Ops.cs:157-165) then RMSNorm of the k row; without
    // the norm the factor is 1 and gamma the ones vector
    float y[8], ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float yv = x[e];
        if constexpr (HK > 0) {
            const float xp = rope_partner_dpp<HK>(x[e], c);
            const bool rot = d0 < 64 * HK, lower = (d0 & rh) == 0;
            yv = !rot ? x[e] : lower ? x[e] * cs[e] - xp * sn[e] : xp * sn[e] + x[e] * cs[e];
        }
        y[e] = yv;
        ss += yv * yv;
    }
    ss = dpp_sum16(ss);
    const float rr = a.norm_k ? 1.0f / sqrtf(ss / (float)D + a.eps) : 1.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = y[e] * rr * gw[e];
    uint32_t kw[4];
#pragma unroll
    for (int e = 0; e < 4; e++) kw[e] = (uint32_t)to_elem<T>(y[2 * e]) | ((uint32_t)to_elem<T>(y[2 * e + 1]) << 16);
    const size_t page_base = ((size_t)phys * Hkv + kvh) * (size_t)(P * D);
    // the barrier precedes every global store: a store issued before it
    // would be waited for at the barrier
    __syncthreads();
    if (valid) *(uint4 *)((S *)a.kpool + page_base + k_off16(pstart % P + r, d0)) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
    // V: thread -> chunk (pc = 4 * (step) + g, d) with d = tid % 128, g = tid / 128:
    // block rows 4g + [0, 4) and 16 + 4g + [0, 4), one 16-byte store.  In the
    // chunk's first block a position before the chunk (pos0 not a multiple
    // of 32) keeps its cached value: those chunks are stored element-wise.
    {
        const int d = tid & (D - 1), g = tid >> 7;
        S *vpage = (S *)a.vpool + page_base + v_off16(pstart % P + 4 * g, d);
        const int rows[8] = {4 * g, 4 * g + 1, 4 * g + 2, 4 * g + 3, 16 + 4 * g, 17 + 4 * g, 18 + 4 * g, 19 + 4 * g};
        if (pstart + 4 * g >= a.pos0) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; e++) w[e] = (uint32_t)s_v[rows[2 * e]][d] | ((uint32_t)s_v[rows[2 * e + 1]][d] << 16);
            *(uint4 *)vpage = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (pstart + rows[e] >= a.pos0) vpage[e] = s_v[rows[e]][d];
        }
    }
}

template <typename T, bool IN_BF16> void launch_kv(const PrepArgs &a, dim3 grid, hipStream_t s) {
    const int hk = a.rope_half >> 5;
    KernelSpan span("prefill_kv", s, true);
    if (hk == 2) launch(span, prefill_kv_kernel<T, IN_BF16, 2>, grid, dim3(512), 0, s, a);
    else if (hk == 1) launch(span, prefill_kv_kernel<T, IN_BF16, 1>, grid, dim3(512), 0, s, a);
    else launch(span, prefill_kv_kernel<T, IN_BF16, 0>, grid, dim3(512), 0, s, a);
}

hipError_t launch_prefill_prep(int kv_dtype, const PrepArgs &a, hipStream_t s) {
    // blocks of 32 positions from the chunk's first to the end of the page
    // holding its last position (the V rows past the chunk are zeroed)
    const int first = a.pos0 & ~31, last = ((a.pos0 + a.seq + kPage - 1) & ~(kPage - 1)) - 1;
    // grid rows [0, kv_heads): k/v; with qready, [kv_heads, kv_heads + heads): q
    dim3 grid((last - first) / 32 + 1, a.kv_heads + (a.qready ? a.heads : 0));
    if (a.rope_dim != 0 && a.rope_dim != 64 && a.rope_dim != 128) return hipErrorInvalidValue;
    switch (kv_dtype) {
    case 1: a.io_bf16 ? launch_kv<F16, true>(a, grid, s) : launch_kv<F16, false>(a, grid, s); break;
    case 2: a.io_bf16 ? launch_kv<BF16, true>(a, grid, s) : launch_kv<BF16, false>(a, grid, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ work items
// A work item is (block pair, kv tile range).  Pairs are enumerated longest
// first; a pair whose range exceeds `cap` tiles is split into
// ceil(tiles/cap) consecutive items.
__host__ __device__ inline int flash_splits(int tiles, int cap) { return (tiles + cap - 1) / cap; }

struct FlashItem {
    int pair, split, nsplit, t0, t1, first;  // `first`: item index of split 0
};

__device__ inline FlashItem flash_item(const FlashArgs &a, int item) {
    FlashItem it;
    if (a.split_ns > 1) {
        // every pair splits alike (a chunk over a long cache): closed form,
        // instead of a scalar loop over the pairs with a division each, which
        // held the first tile copy back 1.3 us at a 256-row chunk over 8192
        const int ns = a.split_ns, pr = item / ns, s = item - pr * ns;
        const int nt = pr < a.npairs ? pair_tiles(a.pos0, pr, a.nb16, a.seq) : 0;
        it.pair = pr < a.npairs ? pr : -1;
        it.split = s;
        it.nsplit = ns;
        it.t0 = s * nt / ns;
        it.t1 = (s + 1) * nt / ns;
        it.first = pr * ns;
        return it;
    }
    if (flash_splits(pair_tiles(a.pos0, 0, a.nb16, a.seq), a.cap) == 1) {
        // pair 0 is the longest: when it is not split no pair is, and item i
        // is pair i
        it.pair = item < a.npairs ? item : -1;
        it.split = 0;
        it.nsplit = 1;
        it.t0 = 0;
        it.t1 = item < a.npairs ? pair_tiles(a.pos0, item, a.nb16, a.seq) : 0;
        it.first = item;
        return it;
    }
    int first = 0;
    for (int pr = 0; pr < a.npairs; pr++) {
        const int nt = pair_tiles(a.pos0, pr, a.nb16, a.seq);
        const int ns = flash_splits(nt, a.cap);
        if (item < first + ns) {
            const int s = item - first;
            it.pair = pr;
            it.split = s;
            it.nsplit = ns;
            it.t0 = s * nt / ns;
            it.t1 = (s + 1) * nt / ns;
            it.first = first;
            return it;
        }
        first += ns;
    }
    it.pair = -1;
    return it;
}

// ------------------------------------------------------------------ flash
template <typename T> struct Mfma;
template <> struct Mfma<BF16> {
    typedef bf16x8 vec;
    __device__ static __forceinline__ f32x4 mma(const vec &a, const vec &b, const f32x4 &c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<F16> {
    typedef f16x8 vec;
    __device__ static __forceinline__ f32x4 mma(const vec &a, const vec &b, const f32x4 &c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// LDS layout of a staged tile.  gfx950 serves a 16-byte LDS access of 16
// lanes in one pass only when lanes 8i..8i+7 cover one 128-byte aligned
// segment and the two 8-lane halves of each 16-lane group sit in opposite
// 128-byte halves of a 256-byte block; any other pattern takes two passes.
// Both tiles are therefore stored as 16-byte chunks in operand order, so that
// every operand read and every staging store is one linear 1 KiB wave access.
// The cache pages already hold their chunks in that order (k_off16 and
// v_off16), so a tile is staged by a straight copy of its two pages:
//   K: chunk (kb, j, c) = dims 8j..8j+7 of position 16 kb + c, at index
//      (kb * 16 + j) * 16 + c;  the S^T A operand of block kb (positions
//      16 kb + [0, 16)), dim step ks, is chunk (kb, 4 ks + grp, c) for lane
//      (grp, c), and the S^T output of lane (grp, c) is positions
//      16 kb + 4 grp + [0, 4).
//   V: chunk (pc, d) at index pc * 128 + d holds positions
//      v_chunk_pos(pc, 0..7) of V^T row d;  the P.V A operand of dim block
//      db, step ks2 is chunk (4 ks2 + grp, 16 db + c) for lane (grp, c), and
//      its positions are the S^T outputs of lane (grp, c) for blocks 2 ks2
//      and 2 ks2 + 1: the P^T B operand of that lane, as packed.


// Row sum of a packed pair of softmax weights (v_dot2c_f32_{bf16,f16} with
// (1, 1)): l accumulates exactly the rounded weights the P*V MFMA uses.
template <typename T> __device__ __forceinline__ float sum2(uint32_t pair, float acc);
template <> __device__ __forceinline__ float sum2<BF16>(uint32_t pair, float acc) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, pair), __builtin_bit_cast(v2, 0x3F803F80u), acc, false);
}
template <> __device__ __forceinline__ float sum2<F16>(uint32_t pair, float acc) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, pair), __builtin_bit_cast(v2, 0x3C003C00u), acc, false);
}

// Staged RoPE rows: float4 (tbl, f4, row) at index (tbl * 16 + f4) * 32 + row
// (tbl 0 = cos, 1 = sin; rows 0..15 block A, 16..31 block B), so the 16 lanes
// that read one dim chunk of 16 rows read one 256-byte block.
constexpr int kRopeF4 = 16;  // float4 per table row (rope_dim / 8 <= 16)

// q rows rowq[qq] + c of head h after RoPE and RMSNorm, times qscale, as the
// S^T B operand: lane (grp, c) holds dims 32*ks + 8*grp + [0, 8).  The RoPE
// partner of dim d (d +- rope_dim/2, rope_dim in {0, 64, 128}) is dim chunk
// ks ^ (rope_dim/64) of the same lane, so no data crosses lanes except the
// norm's sum of squares.  q_load issues the row loads (before the prologue's
// barrier, so they overlap the staging of the first tile); q_finish reads the
// RoPE rows from LDS and builds the operand.  Rows past the chunk or of an
// absent block use q = 0 (their results are discarded).
template <bool IN_BF16> struct QRaw {
    uint4 u[2][4][IN_BF16 ? 1 : 2];
    float4 g[4][2];  // gamma of the lane's dims 32*ks + 8*grp + [0, 8)
};

template <bool IN_BF16>
__device__ __forceinline__ void q_load(const FlashArgs &a, int h, const int (&rowq)[2], const bool (&okq)[2],
                                       int grp, int c, QRaw<IN_BF16> &raw, bool (&ok)[2]) {
    constexpr int D = kHeadDim;
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
        const int row0 = rowq[qq] + c;
        ok[qq] = okq[qq] && row0 < a.seq;
        const int row = min(row0, a.seq - 1);
        const size_t base = (size_t)row * a.q_ld + (size_t)h * D + 8 * grp;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            if (IN_BF16) {
                raw.u[qq][ks][0] = *(const uint4 *)((const uint16_t *)a.q + base + 32 * ks);
            } else {
                raw.u[qq][ks][0] = *(const uint4 *)((const float *)a.q + base + 32 * ks);
                raw.u[qq][ks][IN_BF16 ? 0 : 1] = *(const uint4 *)((const float *)a.q + base + 32 * ks + 4);
            }
        }
    }
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        raw.g[ks][0] = *(const float4 *)(a.qnw + 32 * ks + 8 * grp);
        raw.g[ks][1] = *(const float4 *)(a.qnw + 32 * ks + 8 * grp + 4);
    }
}

// HK = rope_dim / 64: dim chunk ks rotates with chunk ks ^ HK (HK 0: no RoPE).
template <typename T, bool IN_BF16, int HK>
__device__ __forceinline__ void q_finish(const FlashArgs &a, const QRaw<IN_BF16> &raw, const bool (&ok)[2],
                                         int grp, int c, const float *rope_lds, typename Mfma<T>::vec (&qf)[2][4]) {
    constexpr int D = kHeadDim;
    typedef typename Mfma<T>::vec vec;
    const int rh = a.rope_half;
    float gw[4][8];  // gamma: the host passes a ones vector when the norm is off
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const float4 g0 = raw.g[ks][0], g1 = raw.g[ks][1];
        gw[ks][0] = g0.x; gw[ks][1] = g0.y; gw[ks][2] = g0.z; gw[ks][3] = g0.w;
        gw[ks][4] = g1.x; gw[ks][5] = g1.y; gw[ks][6] = g1.z; gw[ks][7] = g1.w;
    }
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
        float x[4][8];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            if (IN_BF16) {
                const uint4 u = raw.u[qq][ks][0];
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[ks][2 * e] = ok[qq] ? __uint_as_float(w[e] << 16) : 0.0f;
                    x[ks][2 * e + 1] = ok[qq] ? __uint_as_float(w[e] & 0xFFFF0000u) : 0.0f;
                }
            } else {
                const uint4 u0 = raw.u[qq][ks][0], u1 = raw.u[qq][ks][IN_BF16 ? 0 : 1];
                const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int e = 0; e < 8; e++) x[ks][e] = ok[qq] ? __uint_as_float(w[e]) : 0.0f;
            }
        }
        float cA[8], cB[8], sA[8], sB[8];
        if (HK) {
            const float4 *rc = (const float4 *)rope_lds + qq * 16 + c;  // row qq*16 + c
            const float4 *rs = rc + kRopeF4 * 32;
            const int fa = ((8 * grp) & (rh - 1)) >> 2, fb = ((32 + 8 * grp) & (rh - 1)) >> 2;
#pragma unroll
            for (int e4 = 0; e4 < 2; e4++) {
                const float4 ca = rc[(fa + e4) * 32];
                const float4 cb = rc[(fb + e4) * 32];
                const float4 sa = rs[(fa + e4) * 32];
                const float4 sb = rs[(fb + e4) * 32];
                cA[4 * e4] = ca.x; cA[4 * e4 + 1] = ca.y; cA[4 * e4 + 2] = ca.z; cA[4 * e4 + 3] = ca.w;
                cB[4 * e4] = cb.x; cB[4 * e4 + 1] = cb.y; cB[4 * e4 + 2] = cb.z; cB[4 * e4 + 3] = cb.w;
                sA[4 * e4] = sa.x; sA[4 * e4 + 1] = sa.y; sA[4 * e4 + 2] = sa.z; sA[4 * e4 + 3] = sa.w;
                sB[4 * e4] = sb.x; sB[4 * e4 + 1] = sb.y; sB[4 * e4 + 2] = sb.z; sB[4 * e4 + 3] = sb.w;
            }
        }
        float y[4][8], ss = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            // RoPE (Ops.RopeRange): first half x*c - x'*s, second half x'*s + x*c
            const bool rot = ks < 2 * HK, lower = (ks & HK) == 0;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float xv = x[ks][e];
                float v = xv;
                if (rot) {
                    const float xp = x[ks ^ HK][e];
                    const float cv = (ks & 1) ? cB[e] : cA[e];
                    const float sv = (ks & 1) ? sB[e] : sA[e];
                    v = lower ? xv * cv - xp * sv : xp * sv + xv * cv;
                }
                y[ks][e] = v;
                ss += v * v;
            }
        }
        const float sum = pf_xrow_sum(ss);
        const float rr = a.norm_q ? 1.0f / sqrtf(sum / (float)D + a.eps) : 1.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[e] = pack2<T>(y[ks][2 * e] * rr * gw[ks][2 * e] * a.qscale,
                                y[ks][2 * e + 1] * rr * gw[ks][2 * e + 1] * a.qscale);
            qf[qq][ks] = __builtin_bit_cast(vec, make_uint4(w[0], w[1], w[2], w[3]));
        }
    }
}

// Instruction order of a 16-read, 16 * (2 - QQ0)-MFMA product (S or P.V of
// one tile): DEPTH LDS reads ahead, then one read after the MFMAs of each
// operand, so that DEPTH reads stay in flight.  Left to itself the scheduler
// keeps one or two reads ahead and each MFMA waits out the LDS latency;
// measured at 2048 tokens, 8 ahead with one MFMA per read (the long block
// alone) and 6 ahead with two (both blocks) are fastest.
template <int QQ0> __device__ __forceinline__ void lds_pipeline() {
    constexpr int DEPTH = QQ0 ? 8 : 6, MPR = 2 - QQ0;
    // masks: 0x100 LDS read, 0x008 MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, DEPTH, 0);
#pragma unroll
    for (int i = 0; i < 16 - DEPTH; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, MPR, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, MPR * DEPTH, 0);
}

// Lazy running maximum: a row's reference m moves only when a tile holds a
// score above m + kLazy (log2 units).  Weights p = 2^(s - m) then stay below
// 2^kLazy and most tiles skip the rescale of O and l entirely.
constexpr float kLazy = 8.0f;

// 8 waves: wave w computes head (w & 3) of the GQA group over the tiles of
// parity (w >> 2) in the item's range, so each SIMD runs two waves.  The
// wave's 32 q rows are the 16 rows of the pair's short block A (qq = 0) and
// the 16 of its long block B (qq = 1); tiles past A's causal range run B
// alone.  Tile pair j sits in LDS buffer j & 1 (one slot per parity); the
// two halves' (m, l, O) are combined through LDS at the end.
template <typename T, bool IN_BF16, int HK, bool PAGES_ARG, bool QREADY>
__global__ __launch_bounds__(512, 1) void prefill_flash_kernel(FlashArgs args) {
    // The arguments pass through one empty asm (scalars as outputs, pointers
    // as inputs, which keeps their global address space): the compiler then
    // issues every argument load in one batch with one wait, instead of
    // waiting on the first few before it issues the rest, and cannot load
    // one again later.
    FlashArgs a = args;
    asm volatile(""
                 : "+s"(a.pos0), "+s"(a.seq), "+s"(a.heads), "+s"(a.kv_heads), "+s"(a.rope_half), "+s"(a.io_bf16),
                   "+s"(a.norm_q), "+s"(a.eps), "+s"(a.qscale), "+s"(a.nb16), "+s"(a.npairs), "+s"(a.cap),
                   "+s"(a.items_per_kvh), "+s"(a.q_ld), "+s"(a.out_bf16)
                 : "s"(a.q), "s"(a.qnw), "s"(a.qready), "s"(a.rope_cos), "s"(a.rope_sin), "s"(a.tab), "s"(a.kpool),
                   "s"(a.vpool), "s"(a.out), "s"(a.part_o), "s"(a.part_ml));
    constexpr int D = kHeadDim, P = kPage, G = kGroup;
    constexpr int KT = P * D;  // elements of one staged K or V tile (16 KiB)
    typedef typename Mfma<T>::vec vec;
    // K slot (buffer, parity) at sKV + (2 * buffer + parity) * KT, its V slot
    // 4 * KT further; sKV doubles as the merge area of the epilogue
    // ([head][17][64] float4 = 69632 bytes)
    __shared__ __attribute__((aligned(16))) uint16_t sKV[8 * KT];
    __shared__ int32_t sTab[kItemTiles];  // physical pages of the item's tiles

    // the wave index is uniform: tile indices, the page ids and the branches
    // on them stay scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hw = wave & 3, half = wave >> 2;
    const int grp = lane >> 4, c = lane & 15;
    const int Hkv = a.kv_heads;

    // XCD-aware placement: workgroup b runs on XCD b % 8; give each XCD one kv
    // head's items so its L2 holds that head's K/V pages.
    const int R = 8 / Hkv;
    const int b = blockIdx.x;
    const int kvh = (b % 8) / R;
    const int item_idx = (b / 8) * R + (b % 8) % R;
    if (item_idx >= a.items_per_kvh) return;
    const FlashItem it = flash_item(a, item_idx);
    const int h = kvh * G + hw;
    // the pair's blocks: qq = 0 -> short block A, qq = 1 -> long block B
    const int blkA = it.pair, blkB = a.nb16 - 1 - it.pair;
    const bool hasA = blkA < blkB;
    const int lenA = hasA ? block_tiles(a.pos0, blkA, a.seq) : 0;  // A attends to tiles [0, lenA)
    const int rowq[2] = {16 * blkA, 16 * blkB};
    const bool okq[2] = {hasA, true};
    const int L = a.pos0 + a.seq;
    const size_t page_elems = (size_t)P * D;
    const uint16_t *kpool = (const uint16_t *)a.kpool;
    const uint16_t *vpool = (const uint16_t *)a.vpool;

    // K/V tile staging: the 4 waves of a parity copy both pages of the
    // parity's tile into its LDS slots with direct global->LDS loads
    // (global_load_lds_dwordx4: lane i writes LDS bytes base + 16 i), wave hw
    // taking chunks (4 i + hw) * 64 + lane of each page, i = 0..3.  The LDS
    // tile is the page verbatim.  V rows past the chunk were zeroed by the k/v
    // kernel, so whole pages are copied.
    const uint32_t lds_kv = __builtin_amdgcn_readfirstlane(lds_addr(sKV) + hw * 1024);
    // page 0 = K, 1 = V of the tile in physical page `phys`
    // (the page base is uniform and goes in SGPRs; the lane's byte offset
    // within each 4 KiB quarter is one VGPR for every copy)
    const uint32_t dma_off = (hw * 64 + lane) * 16;
    auto fetch_page = [&](int phys, int buf, int page) __attribute__((always_inline)) {
        const uint16_t *base =
            (page ? vpool : kpool) + ((size_t)__builtin_amdgcn_readfirstlane(phys) * Hkv + kvh) * page_elems;
        const uint32_t dst = lds_kv + ((page ? 4 : 0) + buf * 2 + half) * KT * 2;
#pragma unroll
        for (int i = 0; i < 4; i++) lds_dma16_sv(base + i * 2048, dma_off, dst + i * 4096);
    };
    auto fetch = [&](int phys, int buf) __attribute__((always_inline)) {
        fetch_page(phys, buf, 0);
        fetch_page(phys, buf, 1);
    };

    // ---- start: every prologue load is issued before the first tile's
    // page copies, in straight-line code -- the item's page ids (up to two
    // per thread), the page id of this wave's first tile, the q rows and
    // gamma, the pair's RoPE rows -- so that waiting for the small ones never
    // waits for the copies (vmcnt retires in order), and they all share one
    // memory round trip.  The RoPE rows go to the LDS slot of tile pair 1,
    // which is first written after iteration 0.
    const int nt = it.t1 - it.t0;  // <= kItemTiles (host caps items)
    static_assert(kItemTiles <= 1024, "two page ids per thread");
    const int tab0 = a.tab[it.t0 + min(tid, nt - 1)];
    const int tab1 = a.tab[it.t0 + min(tid + 512, nt - 1)];
    const int half_u = __builtin_amdgcn_readfirstlane(half);
    // the page of this wave's first tile: from the argument list (a scalar
    // load in the argument batch) when the host passes the pages there, so
    // the first copy waits for no table load
    int phys_first;
    if constexpr (PAGES_ARG) phys_first = args.pages[min(it.t0 + min(half_u, nt - 1), kArgPages - 1)];
    else phys_first = __builtin_amdgcn_readfirstlane(a.tab[it.t0 + min(half_u, nt - 1)]);
    vec qf[2][4];
    if constexpr (QREADY) {
        // the wave's q rows, prepared by prefill_kv, as S^T B operands: lane
        // (grp, c) holds dims 32 ks + 8 grp + [0, 8) of row rowq[qq] + c;
        // rows past the chunk or of an absent block are 0 (results discarded)
        const size_t qrow = (size_t)a.heads * D;
        uint4 qu[2][4];
        bool qok[2];
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int row0 = rowq[qq] + c;
            qok[qq] = okq[qq] && row0 < a.seq;
            const size_t base = (size_t)min(row0, a.seq - 1) * qrow + (size_t)h * D + 8 * grp;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) qu[qq][ks] = *(const uint4 *)(a.qready + base + 32 * ks);
        }
        if (half_u < nt) fetch(phys_first, 0);
        if (tid < nt) sTab[tid] = tab0;
        if (tid + 512 < nt) sTab[tid + 512] = tab1;
#pragma unroll
        for (int qq = 0; qq < 2; qq++)
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
                qf[qq][ks] = __builtin_bit_cast(vec, qok[qq] ? qu[qq][ks] : make_uint4(0, 0, 0, 0));
    } else {
        QRaw<IN_BF16> raw;
        bool qok[2];
        q_load<IN_BF16>(a, h, rowq, okq, grp, c, raw, qok);
        // RoPE rows: float4 (table, 4 dims, row) i = tid + 512 k of 16 * rope_half
        // (k = 0, 1; named values, not an array, which the compiler would place
        // in LDS and store before the tile copies)
        constexpr int RH = 32 * HK;  // rope_half
        auto rope_src = [&](int k) {
            const int i = min(tid + 512 * k, max(16 * RH - 1, 0));
            const int r = i & 31, f4 = RH ? (i >> 5) % (RH / 4) : 0, tbl = RH ? i / (8 * RH) : 0;
            const int row = min((r < 16 ? 16 * blkA : 16 * blkB) + (r & 15), a.seq - 1);
            return (const float4 *)((tbl ? a.rope_sin : a.rope_cos) + (size_t)(a.pos0 + row) * RH + 4 * f4);
        };
        float4 rope_v0 = make_float4(0.f, 0.f, 0.f, 0.f), rope_v1 = rope_v0;
        if constexpr (HK > 0) {
            rope_v0 = *rope_src(0);
            rope_v1 = *rope_src(1);
        }
        // the small loads (page ids, q rows, gamma, RoPE rows) land first, with
        // no tile copy queued behind them; then the first tile's copies go out
        // and the RoPE staging, barrier and q_finish run while they land
        __builtin_amdgcn_s_waitcnt(0);
        if (tid < nt) sTab[tid] = tab0;
        if (tid + 512 < nt) sTab[tid + 512] = tab1;
        // the V slot of buffer 1, parity 0 (16 KiB = 2 * kRopeF4 * 32 float4)
        float *rope_lds = (float *)(sKV + (4 + 2) * KT);
        if constexpr (HK > 0) {
            auto rope_put = [&](int k, float4 v) {
                const int i = tid + 512 * k;
                if (i < 16 * RH) {
                    const int r = i & 31, f4 = (i >> 5) % (RH / 4), tbl = i / (8 * RH);
                    ((float4 *)rope_lds)[(tbl * kRopeF4 + f4) * 32 + r] = v;
                }
            };
            rope_put(0, rope_v0);
            rope_put(1, rope_v1);
        }
        if (half_u < nt) fetch(phys_first, 0);
        __syncthreads();
        q_finish<T, IN_BF16, HK>(a, raw, qok, grp, c, rope_lds, qf);
    }

    f32x4 o[8][2];
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int qq = 0; qq < 2; qq++) o[db][qq] = f32x4{0.f, 0.f, 0.f, 0.f};
    // m starts at the reference's -80 (natural log units); l is this lane's
    // partial row sum (its 16 positions of each tile)
    float mrun[2] = {kFloor2, kFloor2}, lrun[2] = {0.f, 0.f};
    const int qmin[2] = {a.pos0 + rowq[0], a.pos0 + rowq[1]};  // first q position of each block

    __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the first tiles has landed
    __syncthreads();

    // One tile of this wave's parity for q blocks QQ0..1 (QQ0 = 0: both
    // blocks; QQ0 = 1: the long block alone).
    // nphys >= 0: the tile this wave stages next (into buffer buf ^ 1); its
    // K page copy is issued before the S MFMAs, its V page copy after them,
    // so that the copies queue behind work instead of in one burst (against
    // K after S and V after the softmax: config 3's flash kernel 31.9 ->
    // 30.7 us, interleaved runs on one box)
    auto tile_body = [&](auto qq0_tag, auto first_tag, int t, int buf, int nphys) {
        constexpr int QQ0 = decltype(qq0_tag)::value;
        constexpr bool first = decltype(first_tag)::value;
        const uint16_t *kt = sKV + (buf * 2 + half) * KT + lane * 8;
        const uint16_t *vt = sKV + (4 + buf * 2 + half) * KT + grp * 1024 + c * 8;
        // ---- S^T - m = K Q^T - m (64 kv x 16 q per block), accumulated onto
        // -m; the half's first tile starts from 0 and sets m from its scores
        if (nphys >= 0) fetch_page(nphys, buf ^ 1, 0);
        f32x4 sacc[4][2];
#pragma unroll
        for (int qq = QQ0; qq < 2; qq++) {
            const float nm = first ? 0.0f : -mrun[qq];
#pragma unroll
            for (int kb = 0; kb < 4; kb++) sacc[kb][qq] = f32x4{nm, nm, nm, nm};
        }
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                vec kf = __builtin_bit_cast(vec, *(const uint4 *)(kt + kb * 2048 + ks * 512));
#pragma unroll
                for (int qq = QQ0; qq < 2; qq++) sacc[kb][qq] = Mfma<T>::mma(kf, qf[qq][ks], sacc[kb][qq]);
            }
        }
        lds_pipeline<QQ0>();

        if (nphys >= 0) fetch_page(nphys, buf ^ 1, 1);

        // ---- online softmax (column c = q row); the causal mask only
        // touches tiles reaching past a block's first row ----
        const int kvbase = t * P;
#pragma unroll
        for (int qq = QQ0; qq < 2; qq++) {
            if (kvbase + P - 1 > qmin[qq]) {
                const int qpos = qmin[qq] + c;
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (kvbase + 16 * kb + 4 * grp + i > qpos) sacc[kb][qq][i] = -INFINITY;
            }
        }
        float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
        for (int qq = QQ0; qq < 2; qq++) {
            float v = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) v = fmaxf(v, sacc[kb][qq][i]);
            mx[qq] = v;
        }
        if constexpr (first) {
#pragma unroll
            for (int qq = QQ0; qq < 2; qq++) {
                mrun[qq] = fmaxf(pf_xrow_max(mx[qq]), kFloor2);
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int i = 0; i < 4; i++) sacc[kb][qq][i] -= mrun[qq];
            }
        } else if (__any(fmaxf(mx[0], mx[1]) > kLazy)) {
            // move m of every row to its maximum when that is higher
#pragma unroll
            for (int qq = QQ0; qq < 2; qq++) {
                const float d = fmaxf(pf_xrow_max(mx[qq]), 0.0f);
                const float al = __builtin_amdgcn_exp2f(-d);
                mrun[qq] += d;
                lrun[qq] *= al;
#pragma unroll
                for (int db = 0; db < 8; db++) o[db][qq] *= al;
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int i = 0; i < 4; i++) sacc[kb][qq][i] -= d;
            }
        }
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int qq = QQ0; qq < 2; qq++)
#pragma unroll
                for (int i = 0; i < 4; i++) sacc[kb][qq][i] = __builtin_amdgcn_exp2f(sacc[kb][qq][i]);

        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ks2++) {
            vec pf[2];
#pragma unroll
            for (int qq = QQ0; qq < 2; qq++) {
                const f32x4 lo = sacc[2 * ks2][qq], hi = sacc[2 * ks2 + 1][qq];
                const uint4 u = make_uint4(pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3]),
                                           pack2<T>(hi[0], hi[1]), pack2<T>(hi[2], hi[3]));
                lrun[qq] = sum2<T>(u.w, sum2<T>(u.z, sum2<T>(u.y, sum2<T>(u.x, lrun[qq]))));
                pf[qq] = __builtin_bit_cast(vec, u);
            }
#pragma unroll
            for (int db = 0; db < 8; db++) {
                vec vf = __builtin_bit_cast(vec, *(const uint4 *)(vt + ks2 * 4096 + db * 128));
#pragma unroll
                for (int qq = QQ0; qq < 2; qq++) o[db][qq] = Mfma<T>::mma(vf, pf[qq], o[db][qq]);
            }
        }
        lds_pipeline<QQ0>();
    };

    // nbA: the item's tiles (from t0) that hold both blocks (t < lenA).  Tile
    // pairs j < nbA / 2 hold both blocks on both parities; when nbA is odd,
    // pair nbA / 2 holds both on parity 0 and the long block alone on parity
    // 1, and is peeled out of the loops, so that no loop joins the two forms
    // (at such a join the compiler moved O between registers on every
    // iteration); after it the long block runs alone, in a loop of its own
    // where the short block's q rows and scores are dead.
    const int nbA = min(max(0, lenA - it.t0), nt);
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using FT = std::integral_constant<bool, true>;
    using FF = std::integral_constant<bool, false>;
    // the parity's first tile (j = 0) sets m from its scores: peeled, so the
    // loops below carry only the lazy-rescale branch
    {
        const int t = it.t0 + half;
        const int nphys = t + 2 < it.t1 ? sTab[t + 2 - it.t0] : -1;
        if (t < it.t1) {
            if (t < lenA) tile_body(I0{}, FT{}, t, 0, nphys);
            else tile_body(I1{}, FT{}, t, 0, nphys);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
    int j = 1;
    for (; j < (nbA >> 1); j++) {
        const int buf = j & 1;
        const int t = it.t0 + 2 * j + half;  // this wave's tile: t < lenA and t < t1
        // tile t + 2 goes into the other buffer, which every wave finished
        // reading before the previous barrier
        const int nphys = t + 2 < it.t1 ? sTab[t + 2 - it.t0] : -1;
        tile_body(I0{}, FF{}, t, buf, nphys);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of tile t + 2 have landed
        __syncthreads();
    }
    if ((nbA & 1) && j == (nbA >> 1)) {
        const int buf = j & 1;
        const int t = it.t0 + 2 * j + half;
        const int nphys = t + 2 < it.t1 ? sTab[t + 2 - it.t0] : -1;
        if (t < it.t1) {
            if (t < lenA) tile_body(I0{}, FF{}, t, buf, nphys);
            else tile_body(I1{}, FF{}, t, buf, nphys);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        j++;
    }
    for (; 2 * j < nt; j++) {
        const int buf = j & 1;
        const int t = it.t0 + 2 * j + half;
        const int nphys = t + 2 < it.t1 ? sTab[t + 2 - it.t0] : -1;
        if (t < it.t1) tile_body(I1{}, FF{}, t, buf, nphys);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }

    // ---- combine the two parities: half 1 hands (m, l, O) to half 0 ----
    float4 *xo = (float4 *)sKV + hw * 17 * 64 + lane;
    if (half) {
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const f32x4 v = o[db][qq];
                xo[(db * 2 + qq) * 64] = make_float4(v[0], v[1], v[2], v[3]);
            }
        xo[16 * 64] = make_float4(mrun[0], mrun[1], lrun[0], lrun[1]);
    }
    __syncthreads();
    // A split item's partial tile ([G][32][D] of its slot, 32 KiB in one
    // block) is restaged through LDS (past the hand-off above) and written as
    // whole lines, 16 bytes a lane: from the MFMA layout each 8-byte store
    // reached 16 rows, 32 bytes of each (config-4 flash kernel 29.4 -> 28.8
    // us).  The same for the bf16 output rows (1 KiB of 4 heads each) was no
    // faster at config 3.  Rows are padded by 16 bytes against bank
    // conflicts on the restaging stores.
    const bool restage = it.nsplit > 1;
    constexpr int kStage = 36864;          // uint16 offset of the restaging area (72 KiB)
    constexpr int RSP = D + 8;             // partial rows [G][32][D], padded
    uint16_t *st = sKV + kStage;
    static_assert(kStage + G * 32 * RSP <= 8 * KT, "restage");
    const int qdim = a.heads * D;
    const size_t slot = (size_t)kvh * a.items_per_kvh + item_idx;
    if (!half) {
        const float4 ml = xo[16 * 64];
        const float m1[2] = {ml.x, ml.y}, l1[2] = {ml.z, ml.w};
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const float M = fmaxf(mrun[qq], m1[qq]);
            const float a0 = exp2f(mrun[qq] - M), a1 = exp2f(m1[qq] - M);
            mrun[qq] = M;
            lrun[qq] = lrun[qq] * a0 + l1[qq] * a1;
#pragma unroll
            for (int db = 0; db < 8; db++) {
                const float4 v = xo[(db * 2 + qq) * 64];
                o[db][qq] = o[db][qq] * a0 + f32x4{v.x, v.y, v.z, v.w} * a1;
            }
        }

        // ---- finish: row sums across the 4 lane groups ----
#pragma unroll
        for (int qq = 0; qq < 2; qq++) lrun[qq] = pf_xrow_sum(lrun[qq]);
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int r = qq * 16 + c;
            const float inv = lrun[qq] > 0.f ? 1.0f / lrun[qq] : 0.f;
            if (it.nsplit > 1) {
                // split item: O / l rounded to the operand type (the weights sum
                // to 1, so |O / l| <= max |V| fits it), and (m, l) in fp32
#pragma unroll
                for (int db = 0; db < 8; db++) {
                    const f32x4 v = o[db][qq] * inv;
                    *(uint2 *)(st + (hw * 32 + r) * RSP + db * 16 + grp * 4) =
                        make_uint2(pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]));
                }
                if (grp == 0) {
                    float *pm = a.part_ml + ((slot * G + hw) * 32 + r) * 2;
                    pm[0] = mrun[qq];
                    pm[1] = lrun[qq];
                }
            } else {
                const int row = rowq[qq] + c;
                if (!okq[qq] || row >= a.seq) continue;
                const size_t off = (size_t)row * qdim + (size_t)h * D + grp * 4;
                if (a.out_bf16) {
                    uint16_t *orow = (uint16_t *)a.out + off;
#pragma unroll
                    for (int db = 0; db < 8; db++) {
                        const f32x4 v = o[db][qq] * inv;
                        *(uint2 *)(orow + db * 16) =
                            make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                                       (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
                    }
                } else {
                    float *orow = a.out + off;
#pragma unroll
                    for (int db = 0; db < 8; db++) {
                        const f32x4 v = o[db][qq] * inv;
                        *(float4 *)(orow + db * 16) = make_float4(v[0], v[1], v[2], v[3]);
                    }
                }
            }
        }
    }
    if (!restage) return;
    __syncthreads();
    // 32 KiB: [G][32][D] of the item's slot, one contiguous block; 4 chunks
    // of 16 bytes a thread
#pragma unroll
    for (int n = 0; n < 4; n++) {
        const int q = n * 512 + tid, row = q >> 4, col = q & 15;
        *(uint4 *)((uint16_t *)a.part_o + (slot * G * 32 + row) * D + col * 8) =
            *(const uint4 *)(st + row * RSP + col * 8);
    }
}

template <typename T, bool IN_BF16, bool PA> void launch_flash_pa(const FlashArgs &a, dim3 grid, hipStream_t s) {
    const int hk = a.rope_half >> 5;
    KernelSpan span("prefill_flash", s, true);
    if (a.qready) launch(span, prefill_flash_kernel<T, false, 0, PA, true>, grid, dim3(512), 0, s, a);
    else if (hk == 2) launch(span, prefill_flash_kernel<T, IN_BF16, 2, PA, false>, grid, dim3(512), 0, s, a);
    else if (hk == 1) launch(span, prefill_flash_kernel<T, IN_BF16, 1, PA, false>, grid, dim3(512), 0, s, a);
    else launch(span, prefill_flash_kernel<T, IN_BF16, 0, PA, false>, grid, dim3(512), 0, s, a);
}
template <typename T, bool IN_BF16> void launch_flash(const FlashArgs &a, dim3 grid, hipStream_t s) {
    if (a.pages_in_args) launch_flash_pa<T, IN_BF16, true>(a, grid, s);
    else launch_flash_pa<T, IN_BF16, false>(a, grid, s);
}

hipError_t launch_prefill_flash(int kv_dtype, const FlashArgs &a, int total_items, hipStream_t s) {
    (void)total_items;
    const int R = 8 / a.kv_heads;
    const int per_xcd = (a.items_per_kvh + R - 1) / R;
    dim3 grid(per_xcd * 8);
    if (a.rope_dim != 0 && a.rope_dim != 64 && a.rope_dim != 128) return hipErrorInvalidValue;
    switch (kv_dtype) {
    case 1: a.io_bf16 ? launch_flash<F16, true>(a, grid, s) : launch_flash<F16, false>(a, grid, s); break;
    case 2: a.io_bf16 ? launch_flash<BF16, true>(a, grid, s) : launch_flash<BF16, false>(a, grid, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ merge
// Combine the split items of a block pair: one workgroup per (pair, kv head,
// head in group, 8-row quarter of the pair's 32 rows); thread -> (row, 4
// dims).  out = sum_s w_s l_s (O_s / l_s) / sum_s w_s l_s, w_s = 2^(m_s - max
// m).  With at most PER splits every (m, l) and partial row O_s / l_s (type
// T) of the thread is loaded at once, one memory round trip (slots past the
// pair's splits load the last split again and are masked); PER = 0 takes any
// split count, the (m, l) first and then the rows up to 8 at a time.
template <typename T, int PER>
__global__ __launch_bounds__(256) void prefill_merge_kernel(FlashArgs a) {
    constexpr int D = kHeadDim, G = kGroup;
    int b = blockIdx.x;
    const int quarter = b & 3;
    b >>= 2;
    const int g = b % G;
    b /= G;
    const int kvh = b % a.kv_heads;
    const int pr = b / a.kv_heads;
    int first = a.split_ns > 1 ? pr * a.split_ns : 0;
    if (a.split_ns <= 1)
        for (int q = 0; q < pr; q++) first += flash_splits(pair_tiles(a.pos0, q, a.nb16, a.seq), a.cap);
    const int ns = a.split_ns > 1 ? a.split_ns : flash_splits(pair_tiles(a.pos0, pr, a.nb16, a.seq), a.cap);
    if (ns <= 1) return;
    const int r = quarter * 8 + threadIdx.x / 32;  // row of the pair: r < 16 block A, else B
    const int blk = r < 16 ? pr : a.nb16 - 1 - pr;
    if (r < 16 && blk >= a.nb16 - 1 - pr) return;  // the middle block has no A rows
    const int row = blk * 16 + (r & 15);
    if (row >= a.seq) return;
    const int d = (threadIdx.x % 32) * 4;
    const size_t slot0 = (size_t)kvh * a.items_per_kvh + first;
    const float *pm = a.part_ml + ((slot0 * G + g) * 32 + r) * 2;
    const uint16_t *po = (const uint16_t *)a.part_o + ((slot0 * G + g) * 32 + r) * D + d;
    const size_t ml_stride = (size_t)G * 32 * 2, o_stride = (size_t)G * 32 * D;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float Ls = 0.f;
    auto add = [&](float wl, uint2 u) {
        Ls += wl;
        acc.x = fmaf(wl, from_elem<T>((uint16_t)(u.x & 0xFFFF)), acc.x);
        acc.y = fmaf(wl, from_elem<T>((uint16_t)(u.x >> 16)), acc.y);
        acc.z = fmaf(wl, from_elem<T>((uint16_t)(u.y & 0xFFFF)), acc.z);
        acc.w = fmaf(wl, from_elem<T>((uint16_t)(u.y >> 16)), acc.w);
    };
    if constexpr (PER > 0) {
        float2 ml[PER];
        uint2 ov[PER];
#pragma unroll
        for (int s = 0; s < PER; s++) {
            const int ss = min(s, ns - 1);
            ml[s] = *(const float2 *)(pm + ss * ml_stride);
            ov[s] = *(const uint2 *)(po + ss * o_stride);
        }
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < PER; s++) M = fmaxf(M, ml[s].x);  // repeats of the last split change no maximum
#pragma unroll
        for (int s = 0; s < PER; s++)
            if (s < ns) add(exp2f(ml[s].x - M) * ml[s].y, ov[s]);
    } else {
        float M = -INFINITY;
        for (int s = 0; s < ns; s++) M = fmaxf(M, pm[s * ml_stride]);
#pragma unroll 8
        for (int s = 0; s < ns; s++) add(exp2f(pm[s * ml_stride] - M) * pm[s * ml_stride + 1], *(const uint2 *)(po + s * o_stride));
    }
    const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;
    const size_t off = (size_t)row * a.heads * D + (size_t)(kvh * G + g) * D + d;
    if (a.out_bf16)
        *(uint2 *)((uint16_t *)a.out + off) =
            make_uint2((uint32_t)f32_to_bf16(acc.x * inv) | ((uint32_t)f32_to_bf16(acc.y * inv) << 16),
                       (uint32_t)f32_to_bf16(acc.z * inv) | ((uint32_t)f32_to_bf16(acc.w * inv) << 16));
    else
        *(float4 *)(a.out + off) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

template <typename T> void launch_merge(const FlashArgs &a, dim3 grid, hipStream_t s) {
    // the largest split count of any pair (pair 0 is the longest)
    const int ns = flash_splits(pair_tiles(a.pos0, 0, a.nb16, a.seq), a.cap);
    KernelSpan span("prefill_merge", s, true);
    if (ns <= 8) launch(span, prefill_merge_kernel<T, 8>, grid, dim3(256), 0, s, a);
    else if (ns <= 16) launch(span, prefill_merge_kernel<T, 16>, grid, dim3(256), 0, s, a);
    else launch(span, prefill_merge_kernel<T, 0>, grid, dim3(256), 0, s, a);
}

hipError_t launch_prefill_merge(int kv_dtype, const FlashArgs &a, hipStream_t s) {
    const dim3 grid(a.npairs * a.kv_heads * kGroup * 4);
    switch (kv_dtype) {
    case 1: launch_merge<F16>(a, grid, s); break;
    case 2: launch_merge<BF16>(a, grid, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace hymt
