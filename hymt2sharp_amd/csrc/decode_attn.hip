// decode_attn.hip -- fused single-token attention for gfx950.
//
// One launch per layer does what HunyuanDenseModel.DecodeAttention does
// between the QKV GEMV and the O projection (HunyuanDenseModel.Decode.cs:79-95):
//   RoPE q,k at pos (Ops.NeoXRoPE, Ops.cs:98-168) -> RMSNorm q,k (Ops.RmsNorm,
//   Ops.cs:12-90) -> append k,v rounded to the cache dtype (Ops.ConvertToBf16,
//   Ops.cs:658-680) -> softmax(q K^T * scale) V over [0, pos]
//   (Ops.AttentionDecode, Ops.cs:462-532; SoftmaxRow's -80 floor, :224-325).
//
// Work split (flash-decoding, as the reference's Metal attn_split/attn_merge,
// MslDecodeKernels.cs:172-300, but over KV heads so that each K/V byte is read
// from HBM once for all 4 q heads of its GQA group):
//   workgroup = (split, kv head), 4 waves, `ppw` 64-position pages per split
//   (one page per split up to 128 pages, so a 4k-context layer spreads over
//   256 workgroups, every CU; past 256 pages, 128 splits per kv head).
//   Wave w owns 16 positions of every page of its split: those of V chunks 2w
//   and 2w+1 (f16/bf16 pages) or the sub-tile [16w, 16w+16) (f32 pages), so
//   that its K and V operand loads are whole 128-byte segments.
//   The kernel is latency-bound at decode sizes, so the prologue is ordered
//   for the shortest dependent chain: page ids (scalar loads) first, then the
//   q rows, then the K/V stream; no workgroup barrier before the final
//   combine of the 4 wave partials.  Splits are merged by a second launch.
#include <algorithm>
#include <mutex>

#include "attn_kernels.hpp"
#include "device_common.hpp"
#include "ktimer.hpp"

namespace hymt {

typedef float f32x4 __attribute__((ext_vector_type(4)));


// RoPE (Ops.RopeRange, Ops.cs:157-165) of element d of one head row whose
// values at d and at its rotation partner are x and xp.
__device__ __forceinline__ float rope_elem(int d, float x, float xp, float c, float s, int half,
                                           int rope_dim) {
    if (d < half) return x * c - xp * s;
    if (d < rope_dim) return xp * s + x * c;
    return x;
}
__device__ __forceinline__ int rope_partner(int d, int half, int rope_dim) {
    return d < half ? d + half : d < rope_dim ? d - half : d;
}
__device__ __forceinline__ int rope_index(int d, int half, int rope_dim) {
    return d < half ? d : d < rope_dim ? d - half : 0;
}


// ---------------------------------------------------------------------------
// The two dot products run on MFMA.
//   S  = K_sub (16 pos x 128) . Qcat^T      v_mfma_f32_16x16x32_{f16,bf16} x4
//   O += Pcat (16 rows x 16 pos) . V_sub     v_mfma_f32_16x16x16{f16,bf16_1k} x8
// Qcat columns 0..3 hold q of the 4 heads rounded to the operand type and
// columns 4..7 the rounding residual (q - hi) rounded again; Pcat rows 0..3 /
// 4..7 do the same for the softmax weights.  Summing the two halves gives
// q and P to about 2^-22 (f16) or 2^-18 (bf16) relative, i.e. the fp32 path's
// accuracy, with f16/bf16 K and V consumed exactly as stored.  f32 caches use
// the bf16 MFMAs with K and V split the same way (twice the MFMAs).
template <typename T> struct DecMfma;
template <> struct DecMfma<F16> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    typedef _Float16 v4 __attribute__((ext_vector_type(4)));
    __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
    }
    __device__ static __forceinline__ f32x4 pv(uint2 a, uint2 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4, a), __builtin_bit_cast(v4, b), c, 0, 0, 0);
    }
};
template <> struct DecMfma<BF16> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    typedef short v4 __attribute__((ext_vector_type(4)));
    __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
    }
    __device__ static __forceinline__ f32x4 pv(uint2 a, uint2 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4, a), __builtin_bit_cast(v4, b), c, 0, 0, 0);
    }
};

// x split into hi + lo in the operand type: hi = round(x), lo = round(x - hi)
template <typename T> __device__ __forceinline__ uint32_t split_pair(float x) {
    const uint16_t hi = to_elem<T>(x);
    const uint16_t lo = to_elem<T>(x - from_elem<T>(hi));
    return (uint32_t)hi | ((uint32_t)lo << 16);
}

// f32 operands for the bf16 MFMAs: 8 floats (two uint4) -> hi and lo
// operands, x = hi + lo to about 2^-17 relative.
__device__ __forceinline__ void split8(const uint4 &a, const uint4 &b, uint4 &hi, uint4 &lo) {
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t p0 = split_pair<BF16>(__uint_as_float(w[2 * e]));
        const uint32_t p1 = split_pair<BF16>(__uint_as_float(w[2 * e + 1]));
        h[e] = (p0 & 0xFFFFu) | (p1 << 16);
        l[e] = (p0 >> 16) | (p1 & 0xFFFF0000u);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}
// 4 floats of V (positions 4 grp + j) -> hi and lo operands; positions whose
// halfword keep mask is clear are zeroed first
__device__ __forceinline__ void split4(const uint4 &v, const uint32_t (&keep)[2], uint2 &hi, uint2 &lo) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[2], l[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const float x0 = (keep[e] & 0xFFFFu) ? __uint_as_float(w[2 * e]) : 0.0f;
        const float x1 = (keep[e] & 0xFFFF0000u) ? __uint_as_float(w[2 * e + 1]) : 0.0f;
        const uint32_t p0 = split_pair<BF16>(x0), p1 = split_pair<BF16>(x1);
        h[e] = (p0 & 0xFFFFu) | (p1 << 16);
        l[e] = (p0 >> 16) | (p1 & 0xFFFF0000u);
    }
    hi = make_uint2(h[0], h[1]);
    lo = make_uint2(l[0], l[1]);
}

// Cross-row sums / maxima (rows are 16 lanes): permlane swaps on gfx950.
__device__ __forceinline__ float xrow16_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xrow32_sum(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xrow16_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xrow32_max(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// lane i of each 16-lane row receives lane i+4 (row_shl:4) / lane i-4 (row_shr:4)
__device__ __forceinline__ float dpp_from_plus4(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t dpp_from_minus4(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);
}

// Sum over all 64 lanes on the VALU: DPP within 16-lane rows, then the
// row swaps (no LDS round trip).
__device__ __forceinline__ float wave_sum64(float v) { return xrow32_sum(xrow16_sum(dpp_sum16(v))); }

// NR consecutive head rows (q heads of one GQA group, or one k row) held as
// lanes (d, d+64).  All loads -- rows, rotation partners, cos/sin, gamma --
// are issued by load() before any use, unconditionally (the host passes a
// ones vector for an absent gamma or RoPE table), so the kernel's prologue is
// straight-line code: one batch of scalar argument loads, then every vector
// load in one memory round trip.  finish() applies RoPE then RMSNorm
// (HunyuanDenseModel.Decode.cs:80-85).
// FULL: rotary width 128 (half 64), the partner of d is d^64 in the same
// lane and no partner loads are needed.
template <int NR, bool FULL> struct RowsIn {
    float x[NR][2], xp[NR][2], c[2], s[2], w[2];
    __device__ __forceinline__ void load(const float *rows, const float *cosr, const float *sinr,
                                         const float *gamma, int lane, int half, int rdim) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            x[r][0] = rows[r * kHeadDim + lane];
            x[r][1] = rows[r * kHeadDim + lane + 64];
        }
        w[0] = gamma[lane];
        w[1] = gamma[lane + 64];
        if constexpr (FULL) {
            c[0] = c[1] = cosr[lane];
            s[0] = s[1] = sinr[lane];
        } else {
            // partner index d and table index 0 when d is not rotated (the
            // values are then unused)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
#pragma unroll
                for (int r = 0; r < NR; r++) xp[r][e] = rows[r * kHeadDim + rope_partner(d, half, rdim)];
                c[e] = cosr[rope_index(d, half, rdim)];
                s[e] = sinr[rope_index(d, half, rdim)];
            }
        }
    }
    // Row r: RoPE (Ops.cs:157-165) then y = x * (1/sqrt(sum x^2/D + eps)) * gamma
    // (Ops.cs:62-88), times `scale`.  Without the norm the factor is 1 and
    // gamma the ones vector, so y = x exactly; gamma is used on both paths so
    // that its loads stay ahead of the K/V stream (a load used only under a
    // branch is sunk behind it, and vmcnt retires in order).
    __device__ __forceinline__ void finish(int r, float (&y)[2], int lane, int half, int rdim, bool norm,
                                           float eps, float scale) const {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float p = FULL ? x[r][1 - e] : xp[r][e];
            y[e] = FULL ? (e == 0 ? x[r][0] * c[0] - p * s[0] : p * s[1] + x[r][1] * c[1])
                        : rope_elem(lane + 64 * e, x[r][e], p, c[e], s[e], half, rdim);
        }
        const float ss = wave_sum64(y[0] * y[0] + y[1] * y[1]);
        const float rr = norm ? 1.0f / sqrtf(ss / (float)kHeadDim + eps) : 1.0f;
        y[0] = y[0] * rr * w[0];
        y[1] = y[1] * rr * w[1];
        y[0] *= scale;
        y[1] *= scale;
    }
};

// K and V operands of one wave for one page: its 16 positions.
//   f16/bf16 pages: wave w takes the 16 positions of V chunks 2w and 2w+1, so
//   that its V loads are whole 16-byte chunks; S row / P.V index 4 grp + i
//   of the wave is page position posw(i).
//   K A-operand: lane (grp, c) = K row c (position posw of index c), dims
//     32*ks + 8*grp + [0, 8): two 128-byte segments per 16 lanes.
//   V B-operand: lane (grp, c) = V^T row 16*db + c, indices 4*grp + [0, 4):
//     half (grp & 1) of V chunk (2 w + (grp >> 1), 16 db + c).  The lane
//     loads whole 16-byte chunks (those of its row parity's db) and swaps
//     halves with the partner row, so every K and V load is 16 bytes:
//     1.0 % less time per config-2 call and 1.2 % at 32k positions than 8-byte
//     half-chunk loads, the same bytes and cache lines.
//   f32 pages (row-major K, V^T sub-tiles [16w, 16w+16)): the same operands
//   as fp32, two 16-byte K loads per ks and one 16-byte V load per db.
template <typename S> struct PageOps {
    static constexpr bool W4 = sizeof(S) == 4;
    static constexpr int KL = W4 ? 8 : 4;
    uint4 k[KL];
    // V: f32 pages one 16-byte load per db; 16-bit pages the whole chunks of
    // dims 16 db + c for db of the lane's row parity (grp & 1), 4 x 16 bytes,
    // whose other halves the partner row takes (v_halves)
    uint4 v[W4 ? 8 : 4];
    __device__ __forceinline__ void load_k(const S *kpool, size_t pb, int wave, int grp, int c) {
        constexpr int D = kHeadDim, SUB = 16;
        if constexpr (W4) {
            const S *kp = kpool + pb + (size_t)(SUB * wave + c) * D + 8 * grp;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                k[2 * ks] = *(const uint4 *)(kp + 32 * ks);
                k[2 * ks + 1] = *(const uint4 *)(kp + 32 * ks + 4);
            }
        } else {
            const S *kp = kpool + pb + 2048 * (2 * (wave >> 1) + ((c >> 2) & 1)) + 128 * grp +
                          8 * (8 * (wave & 1) + 4 * (c >> 3) + (c & 3));
#pragma unroll
            for (int ks = 0; ks < 4; ks++) k[ks] = *(const uint4 *)(kp + 512 * ks);
        }
    }
    __device__ __forceinline__ void load_v(const S *vpool, size_t pb, int wave, int grp, int c) {
        constexpr int D = kHeadDim, SUB = 16;
        if constexpr (W4) {
            const S *vp = vpool + pb + (size_t)(wave * D + c) * SUB + 4 * grp;
#pragma unroll
            for (int db = 0; db < 8; db++) v[db] = *(const uint4 *)(vp + 256 * db);
        } else {
            const S *vp = vpool + pb + (size_t)(2 * wave + (grp >> 1)) * 1024 + 8 * c + 128 * (grp & 1);
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = *(const uint4 *)(vp + 256 * j);
        }
    }
    // 16-bit pages: the P.V B operands (4 positions of dim 16 db + c, the
    // half grp & 1 of its chunk) from the loaded chunks.  Rows 0/1 (and 2/3)
    // of the wave hold the chunks of even / odd db; one permlane16 swap per
    // dword pair hands each row the halves it lacks: afterwards the first
    // operand holds db = 2 j and the second db = 2 j + 1 in every row.
    __device__ __forceinline__ void v_halves(uint2 (&o)[8]) const {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const auto a = __builtin_amdgcn_permlane16_swap(v[j].x, v[j].z, false, false);
            const auto b = __builtin_amdgcn_permlane16_swap(v[j].y, v[j].w, false, false);
            o[2 * j] = make_uint2(a[0], b[0]);
            o[2 * j + 1] = make_uint2(a[1], b[1]);
        }
    }
    __device__ __forceinline__ void load(const S *kpool, const S *vpool, size_t pb, int wave, int grp, int c) {
        load_k(kpool, pb, wave, grp, c);
        load_v(vpool, pb, wave, grp, c);
    }
};

// Decode for every cache type.
//   The cached positions [0, pos) are split by pages: workgroup (split, kv
//   head), 4 waves, PPW pages per split whose K/V loads are all issued at
//   once; wave w streams 16 positions of each page (PageOps).  For each page
//     S = K_sub . Qcat^T, lane (grp, c<4) gets head c at positions 4*grp + i
//     (its hi part; lanes c+4 hold the lo part).
//   then one softmax over all the split's positions of the wave, then for
//   each page
//     O += Pcat . V_sub, lane (grp, c) gets rows 4*grp + i of dims 16*db + c,
//     rows 0-3 = hi(P) of the 4 heads, rows 4-7 = lo(P).
//   A split of more than PPW pages runs its pages PPW at a time, merging the
//   runs online; the next run's K loads are issued once this run's scores
//   are in (its K registers are free), its V loads after this run's P.V.
//   The new token (position pos) is one more position, handled in the last
//   split on the VALU from registers while the K/V stream is in flight: wave
//   w computes the new K row after RoPE + norm and V, both rounded to the
//   cache type as the reference reads them back from its cache, and head w's
//   weight for it, a fifth partial of the split's combine; wave 0 appends the
//   row to the cache at the end.  So no workgroup is spent on a page that
//   holds only the new token (L = 4097 runs exactly 256 workgroups).
// PAGES_ARG: page ids come from the kernel arguments, else from the device
// page table; both are scalar loads issued first.
template <typename T, int PPW, bool RUNS, bool PAGES_ARG, bool FULL>
__global__ __launch_bounds__(256) void decode_attn_mfma_kernel(DecodeArgs a) {
    constexpr int D = kHeadDim, G = kGroup, P = kPage, SUB = 16;
    // f32 pages: each K and V operand is split on the fly into bf16 hi + lo
    // (x - hi rounded again) and both parts go through the MFMA, so K and V
    // enter the products to about 2^-17 relative, as q and P do
    constexpr bool W4 = sizeof(typename T::storage) == 4;
    using Op = typename std::conditional<W4, BF16, T>::type;  // MFMA operand type
    using M = DecMfma<Op>;
    using S = typename T::storage;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, c = lane & 15;  // MFMA lane group / row-col index
    const int split = blockIdx.x, kvh = blockIdx.y;  // grid (nsplit, kv heads)

    __shared__ __attribute__((aligned(16))) uint16_t s_qop[2][G][D];  // hi/lo q of the 4 heads
    __shared__ __attribute__((aligned(16))) float s_o[4][2][D][G];    // per wave: hi/lo rows
    __shared__ __attribute__((aligned(16))) float s_xo[D][G];         // the new token
    __shared__ float s_m[5][G], s_l[5][G];                             // [4]: the new token

    // ---- 0. the arguments: one batch of scalar loads and one wait ---------
    // Every argument passes through one empty asm as an output.  The compiler
    // must then issue all their loads (page ids from the argument list
    // included: without RUNS a split's pages are PPW consecutive blocks from
    // split * PPW, an address that hangs on blockIdx alone) before the asm
    // and cannot move work on any of them above it, nor load one again later;
    // left to itself it waits on some of them before issuing the rest, and
    // every such scalar round trip delays the K/V stream.
    const S *kpool = (const S *)a.kpool, *vpool = (const S *)a.vpool;
    const float *q_in = a.q, *k_in = a.knew, *v_in = a.vnew, *qnw = a.qnw, *knw = a.knw;
    const float *rcos = a.rope_cos, *rsin = a.rope_sin;
    const int32_t *tab = a.tab;
    float *out_p = a.out, *pml_p = a.part_ml, *pacc_p = a.part_acc;
    int L = a.L, Hkv = a.kv_heads, ppw = RUNS ? a.ppw : PPW, nsplit = a.nsplit;
    int half = a.rope_half, rdim = a.rope_dim, norm_q = a.norm_q, norm_k = a.norm_k;
    float eps = a.eps, qscale = a.qscale;
    // page ids of the split's first PPW pages from the argument list; past
    // its end the index is clamped (the host pads the list with a mapped page)
    int pid[4] = {0, 0, 0, 0};
    if constexpr (PAGES_ARG) {
#pragma unroll
        for (int p = 0; p < PPW; p++) pid[p] = a.pages[min(split * PPW + p, kArgPages - 1)];
    }
    // Pointers that vector loads use are inputs only: an asm output would be
    // a pointer of unknown address space, read by flat loads.  The stores at
    // the end go through global-address-space copies of their pointers.
    asm volatile(""
                 : "+s"(out_p), "+s"(pml_p), "+s"(pacc_p), "+s"(L), "+s"(Hkv), "+s"(ppw), "+s"(nsplit), "+s"(half),
                   "+s"(rdim), "+s"(norm_q), "+s"(norm_k), "+s"(eps), "+s"(qscale), "+s"(pid[0]), "+s"(pid[1]),
                   "+s"(pid[2]), "+s"(pid[3])
                 : "s"(kpool), "s"(vpool), "s"(q_in), "s"(k_in), "s"(v_in), "s"(qnw), "s"(knw), "s"(rcos), "s"(rsin),
                   "s"(tab));
    using gfloat = __attribute__((address_space(1))) float;
    gfloat *out_g = (gfloat *)out_p, *pml_g = (gfloat *)pml_p, *pacc_g = (gfloat *)pacc_p;

    const int newpos = L - 1;                // cached positions [0, newpos)
    const int ncp = (newpos + P - 1) / P;    // cached pages
    const int page0 = split * ppw;
    const int page_end = min(page0 + ppw, ncp);
    const int plast = max(page_end - 1, page0);
    const bool last = split == nsplit - 1;
    const size_t page_elems = (size_t)P * D;
    // a page of the device table (wave-uniform), clamped to the split
    auto tab_page = [&](int p) { return __builtin_amdgcn_readfirstlane(tab[min(p, plast)]); };
    auto page_base = [&](int phys) { return ((size_t)phys * Hkv + kvh) * page_elems; };

    // ---- 1. every vector load, straight-line: the q row of head kvh*4 +
    // wave, the new k and v rows, then the K/V of the split's first PPW
    // pages.  vmcnt retires in order, so the small rows come first: the q
    // operand is built while the stream is in flight.  Pages past the split
    // are read and masked out (with no cached page, pos = 0, the page of pos
    // is read and ignored).
    RowsIn<1, FULL> qin, kin;
    qin.load(q_in + (size_t)(kvh * G + wave) * D, rcos, rsin, qnw, lane, half, rdim);
    kin.load(k_in + (size_t)kvh * D, rcos, rsin, knw, lane, half, rdim);
    const float vnew0 = v_in[(size_t)kvh * D + lane];
    const float vnew1 = v_in[(size_t)kvh * D + lane + 64];
    // the new token's page, whose index hangs on L: from the device table
    // in the same round trip as the split's page ids, from the argument
    // list while the stream is in flight
    int phys_new = 0;
    if constexpr (!PAGES_ARG) phys_new = __builtin_amdgcn_readfirstlane(tab[newpos / P]);
    PageOps<S> pg[PPW];
#pragma unroll
    for (int p = 0; p < PPW; p++)
        pg[p].load(kpool, vpool, page_base(PAGES_ARG ? pid[p] : tab_page(page0 + p)), wave, grp, c);
    if constexpr (PAGES_ARG) {
        phys_new = a.pages[newpos / P];
        asm volatile("" : "+s"(phys_new));
    }

    // ---- 2. q operand: wave w applies RoPE + norm to head w and stores its
    // hi/lo split in LDS; one barrier shares the 4 heads ---------------------
    float qy[2];
    qin.finish(0, qy, lane, half, rdim, norm_q != 0, eps, qscale);
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t pr = split_pair<Op>(qy[e]);
        s_qop[0][wave][lane + 64 * e] = (uint16_t)pr;
        s_qop[1][wave][lane + 64 * e] = (uint16_t)(pr >> 16);
    }

    // ---- 3. the new token (last split): K after RoPE + norm and V, rounded
    // to the cache type (Ops.ConvertToBf16, Ops.cs:658-680), then head w's
    // weight for it in the softmax's base-2 units: m = max(s, floor),
    // l = exp2(max(s - m, floor)).  Its cache stores are issued at the end:
    // vmcnt retires in order, so stores issued here would hold up every
    // later wait on the K/V stream.
    S knew_st[2] = {}, vnew_st[2] = {};
    if (last) {
        float ky[2];
        kin.finish(0, ky, lane, half, rdim, norm_k != 0, eps, 1.0f);
        knew_st[0] = to_elem<T>(ky[0]);
        knew_st[1] = to_elem<T>(ky[1]);
        vnew_st[0] = to_elem<T>(vnew0);
        vnew_st[1] = to_elem<T>(vnew1);
        const float k0 = from_elem<T>(knew_st[0]), k1 = from_elem<T>(knew_st[1]);
        const float sc = wave_sum64(qy[0] * k0 + qy[1] * k1);
        const float m = fmaxf(sc, kFloor2);
        const float l = exp2f(fmaxf(sc - m, kFloor2));
        s_xo[lane][wave] = l * from_elem<T>(vnew_st[0]);
        s_xo[lane + 64][wave] = l * from_elem<T>(vnew_st[1]);
        if (lane == 0) {
            s_m[4][wave] = m;
            s_l[4][wave] = l;
        }
    }
    __syncthreads();
    // Qcat B-operand: lane (grp, c), dims 32*ks + 8*grp + [0, 8):
    // c < 4 -> hi(q_c), 4 <= c < 8 -> lo(q_{c-4}), else 0
    uint4 qb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
        qb[ks] = c < 8 ? *(const uint4 *)&s_qop[c >> 2][c & 3][32 * ks + 8 * grp] : make_uint4(0, 0, 0, 0);

    // ---- 4. attention over the split's cached pages, PPW at a time ---------
    // page position of S row / P.V index 4 grp + i of this wave, and the
    // smallest one
    auto posw = [&](int i) {
        return W4 ? SUB * wave + 4 * grp + i
                  : 32 * (wave >> 1) + 8 * (wave & 1) + 4 * (grp >> 1) + 16 * (grp & 1) + i;
    };
    f32x4 acc[8];
#pragma unroll
    for (int db = 0; db < 8; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kFloor2, l_run = 0.0f;  // lanes c < 4: head c

    for (int run0 = page0; run0 < page_end; run0 += PPW) {
        // scores of the run's pages (positions at or past pos masked out)
        float sc[PPW][4], mt = kFloor2;
#pragma unroll
        for (int p = 0; p < PPW; p++) {
            const int nv = newpos - (run0 + p) * P;  // positions of page p below pos
            f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                if constexpr (W4) {
                    uint4 hi, lo;
                    split8(pg[p].k[2 * ks], pg[p].k[2 * ks + 1], hi, lo);
                    sacc = M::qk(hi, qb[ks], sacc);
                    sacc = M::qk(lo, qb[ks], sacc);
                } else {
                    sacc = M::qk(pg[p].k[ks], qb[ks], sacc);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[p][i] = sacc[i] + dpp_from_plus4(sacc[i]);
                if (run0 + p < page_end && posw(i) < nv) mt = fmaxf(mt, sc[p][i]);
                else sc[p][i] = -INFINITY;
            }
        }
        // the next run's K while this run's softmax and P.V proceed
        size_t nb[PPW];
        const bool more = RUNS && run0 + PPW < page_end;
        if (more) {
#pragma unroll
            for (int p = 0; p < PPW; p++) nb[p] = page_base(tab_page(run0 + PPW + p));
#pragma unroll
            for (int p = 0; p < PPW; p++) pg[p].load_k(kpool, nb[p], wave, grp, c);
        }
        mt = xrow32_max(xrow16_max(mt));
        const float mnew = fmaxf(m_run, mt);
        const float alpha = exp2f(m_run - mnew);
        float pr[PPW][4], ps = 0.0f;
#pragma unroll
        for (int p = 0; p < PPW; p++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pr[p][i] = sc[p][i] == -INFINITY ? 0.0f : exp2f(fmaxf(sc[p][i] - mnew, kFloor2));
                ps += pr[p][i];
            }
        ps = xrow32_sum(xrow16_sum(ps));
        l_run = l_run * alpha + ps;
        m_run = mnew;
        if (run0 != page0) {  // rescale the running sums of earlier runs
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; i++) al[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), i));
#pragma unroll
            for (int db = 0; db < 8; db++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[db][i] *= al[i];
        }
#pragma unroll
        for (int p = 0; p < PPW; p++) {
            // Pcat A-operand: lane (grp, r): r<4 hi(p_r), 4<=r<8 lo(p_{r-4})
            uint32_t hp[2], lp[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t p0 = split_pair<Op>(pr[p][2 * e]), p1 = split_pair<Op>(pr[p][2 * e + 1]);
                hp[e] = (p0 & 0xFFFFu) | (p1 << 16);
                lp[e] = dpp_from_minus4((p0 >> 16) | (p1 & 0xFFFF0000u));
            }
            const uint2 pa = c < 4 ? make_uint2(hp[0], hp[1]) : c < 8 ? make_uint2(lp[0], lp[1]) : make_uint2(0u, 0u);
            // V: zero the positions at or past pos (halfword masks of this
            // lane's 4 positions); they may hold stale data
            const int nv = newpos - (run0 + p) * P;
            uint32_t keep[2] = {0xFFFFFFFFu, 0xFFFFFFFFu};
            if (nv < P) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (posw(j) >= nv) keep[j >> 1] &= ~(0xFFFFu << (16 * (j & 1)));
            }
            if (run0 + p >= page_end) keep[0] = keep[1] = 0u;
            if constexpr (W4) {
#pragma unroll
                for (int db = 0; db < 8; db++) {
                    uint2 hi, lo;
                    split4(pg[p].v[db], keep, hi, lo);
                    acc[db] = M::pv(pa, hi, acc[db]);
                    acc[db] = M::pv(pa, lo, acc[db]);
                }
            } else {
                uint2 vh[8];
                pg[p].v_halves(vh);
#pragma unroll
                for (int db = 0; db < 8; db++)
                    acc[db] = M::pv(pa, make_uint2(vh[db].x & keep[0], vh[db].y & keep[1]), acc[db]);
            }
        }
        // the next run's V (splits of more than PPW pages)
        if (more) {
#pragma unroll
            for (int p = 0; p < PPW; p++) pg[p].load_v(vpool, nb[p], wave, grp, c);
        }
    }

    // ---- 5. combine the wave partials (and the new token) ------------------
    // rows 0-3 (grp 0, hi) and 4-7 (grp 1, lo) of every dim go to LDS as
    // 16-byte vectors [wave][part][dim][head]; (m, l) of head c from lane c.
    if (grp < 2) {
#pragma unroll
        for (int db = 0; db < 8; db++) *(f32x4 *)&s_o[wave][grp][16 * db + c][0] = acc[db];
    }
    if (lane < G) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = l_run;
    }
    __syncthreads();
    {
        const int d = tid & 127, gp = 2 * (tid >> 7);  // thread -> dim d, heads gp, gp+1
        const int nw = last ? 5 : 4;
        float Mx[2], Lx[2] = {0.f, 0.f}, O[2] = {0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; j++) {
            Mx[j] = s_m[0][gp + j];
#pragma unroll
            for (int w = 1; w < 5; w++)
                if (w < nw) Mx[j] = fmaxf(Mx[j], s_m[w][gp + j]);
        }
#pragma unroll
        for (int w = 0; w < 5; w++) {
            if (w >= nw) break;
            float2 o;
            if (w < 4) {
                const float2 hi = *(const float2 *)&s_o[w][0][d][gp];
                const float2 lo = *(const float2 *)&s_o[w][1][d][gp];
                o = make_float2(hi.x + lo.x, hi.y + lo.y);
            } else {
                o = *(const float2 *)&s_xo[d][gp];
            }
            const float sc0 = exp2f(s_m[w][gp] - Mx[0]), sc1 = exp2f(s_m[w][gp + 1] - Mx[1]);
            Lx[0] = fmaf(sc0, s_l[w][gp], Lx[0]);
            Lx[1] = fmaf(sc1, s_l[w][gp + 1], Lx[1]);
            O[0] = fmaf(sc0, o.x, O[0]);
            O[1] = fmaf(sc1, o.y, O[1]);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int h = kvh * G + gp + j;
            if (nsplit == 1) {
                out_g[(size_t)h * D + d] = Lx[j] > 0.0f ? O[j] / Lx[j] : 0.0f;
            } else {
                pacc_g[((size_t)h * kMaxSplits + split) * D + d] = O[j];
                if (d == 0) {
                    gfloat *m = pml_g + ((size_t)h * kMaxSplits + split) * 2;
                    m[0] = Mx[j];
                    m[1] = Lx[j];
                }
            }
        }
    }
    // ---- 6. append the new row to the cache ---------------------------------
    if (last && wave == 0) {
        const int t = newpos % P;
        S *kp = (S *)kpool + ((size_t)phys_new * Hkv + kvh) * page_elems;
        S *vp = (S *)vpool + ((size_t)phys_new * Hkv + kvh) * page_elems;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            kp[k_off<sizeof(S)>(t, lane + 64 * e)] = knew_st[e];
            vp[v_off<sizeof(S)>(t, lane + 64 * e)] = vnew_st[e];
        }
    }
}

// Merge of the split partials (the second launch of a multi-split call):
// out[h] = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s, M = max_s m_s.
// Workgroup = (q head, 32-dim quarter), 256 threads; thread = (split group
// sg of 32, 4 dims d4 of the quarter) over splits sg + 32 k, k < PER
// (32 * PER >= nsplit), so 64 workgroups share the partials' reads and each
// thread issues at most 8 + 8 loads, all at once.  The split groups combine
// within each wave by lane swaps, then the 4 waves through LDS.
struct MergeArgs {
    const float *part_ml;
    const float *part_acc;
    float *out;
    int nsplit;
};
// (m, l, o) += (m2, l2, o2) in base 2: both rescaled to the larger maximum
__device__ __forceinline__ void merge_pair(float &m, float &l, float4 &o, float m2, float l2, float4 o2) {
    const float M = fmaxf(m, m2);
    const float w1 = M == -INFINITY ? 0.0f : exp2f(m - M), w2 = M == -INFINITY ? 0.0f : exp2f(m2 - M);
    m = M;
    l = l * w1 + l2 * w2;
    o = make_float4(o.x * w1 + o2.x * w2, o.y * w1 + o2.y * w2, o.z * w1 + o2.z * w2, o.w * w1 + o2.w * w2);
}
template <int PER>
__global__ __launch_bounds__(256) void decode_merge_kernel(MergeArgs a) {
    constexpr int D = kHeadDim, SG = 32;
    static_assert(SG * PER <= kMaxSplits, "slots past the workspace");
    const int h = blockIdx.x, qd = blockIdx.y, d4 = threadIdx.x & 7, sg = threadIdx.x >> 3;
    const int wave = threadIdx.x >> 6;
    __shared__ float s_m[4][8], s_l[4][8];
    __shared__ float4 s_o[4][8];
    const float2 *ml = (const float2 *)(a.part_ml + (size_t)h * kMaxSplits * 2);
    const float4 *pa = (const float4 *)(a.part_acc + (size_t)h * kMaxSplits * D) + qd * 8 + d4;
    // Every slot is loaded (the workspace holds kMaxSplits per head; slots at
    // or past nsplit hold stale data) and then masked: a load under a
    // condition would be followed by a wait before the next one is issued.
    float2 mlv[PER];
    float4 x[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int s = sg + SG * k;
        mlv[k] = ml[s];
        x[k] = pa[(size_t)s * (D / 4)];
    }
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const bool ok = sg + SG * k < a.nsplit;
        mlv[k] = ok ? mlv[k] : make_float2(-INFINITY, 0.0f);
        x[k] = ok ? x[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float Mv = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; k++) Mv = fmaxf(Mv, mlv[k].x);
    float L = 0.0f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    if (Mv != -INFINITY) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const float w = exp2f(mlv[k].x - Mv);
            L = fmaf(w, mlv[k].y, L);
            O.x = fmaf(w, x[k].x, O.x);
            O.y = fmaf(w, x[k].y, O.y);
            O.z = fmaf(w, x[k].z, O.z);
            O.w = fmaf(w, x[k].w, O.w);
        }
    }
    // the wave's 8 split groups (lanes d4 + 8 j): swaps across 8, 16, 32 lanes
#pragma unroll
    for (int sh = 8; sh < 64; sh <<= 1) {
        const float m2 = __shfl_xor(Mv, sh), l2 = __shfl_xor(L, sh);
        const float4 o2 = make_float4(__shfl_xor(O.x, sh), __shfl_xor(O.y, sh), __shfl_xor(O.z, sh),
                                      __shfl_xor(O.w, sh));
        merge_pair(Mv, L, O, m2, l2, o2);
    }
    if ((threadIdx.x & 63) < 8) {
        s_m[wave][d4] = Mv;
        s_l[wave][d4] = L;
        s_o[wave][d4] = O;
    }
    __syncthreads();
    if (threadIdx.x < 8) {
#pragma unroll
        for (int w = 1; w < 4; w++) merge_pair(Mv, L, O, s_m[w][d4], s_l[w][d4], s_o[w][d4]);
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        ((float4 *)(a.out + (size_t)h * D))[qd * 8 + d4] = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
    }
}

// ---- the decode workspace of hymt_attn_decode_noalloc ------------------------
// A file-scope device array holds the split partials -- (m, l) then acc, laid
// out as DecodeArgs.part_ml / part_acc for up to kScratchHeads q heads -- so
// that a decode call needs no device allocation.  Every GPU that loads the
// library holds its own copy until the process ends; its address on a
// device comes from hipGetSymbolAddress with that device current (in host
// code the array's name is not a device address).  The splits overwrite
// every partial the merge reads, so nothing needs clearing.  One context at
// a time owns a device's array (decode_scratch_claim): its calls run in its
// stream's order, and another context's calls are refused until the owner is
// destroyed.
constexpr int kScratchHeads = 32;
constexpr size_t kScratchMl = (size_t)kScratchHeads * kMaxSplits * 2;        // floats
constexpr size_t kScratchAcc = (size_t)kScratchHeads * kMaxSplits * kHeadDim;  // floats
static __device__ __align__(256) float scratch[kScratchMl + kScratchAcc];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch[kScratchDevices] = {};
// the context whose calls use a device's array (nullptr: none yet); another
// context is refused until the owner releases it, so two contexts' calls can
// never overwrite each other's partials
const void *g_scratch_owner[kScratchDevices] = {};
}  // namespace

bool decode_scratch_claim(int device, const void *owner) {
    if (device < 0 || device >= kScratchDevices || !owner) return false;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_owner[device] && g_scratch_owner[device] != owner) return false;
    g_scratch_owner[device] = owner;
    return true;
}

void decode_scratch_release(int device, const void *owner) {
    if (device < 0 || device >= kScratchDevices) return;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_owner[device] == owner) g_scratch_owner[device] = nullptr;
}

hipError_t decode_scratch_init(int device) {
    if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[device]) return hipSuccess;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));  // the current device's copy
    if (e != hipSuccess) return e;
    g_scratch[device] = (float *)ptr;
    return hipSuccess;
}

hipError_t decode_scratch(int device, float **part_ml, float **part_acc, int *max_heads) {
    if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    float *p = g_scratch[device];
    if (!p) return hipErrorNotInitialized;
    *part_ml = p;
    *part_acc = p + kScratchMl;
    *max_heads = kScratchHeads;
    return hipSuccess;
}

using DecodeKernel = void (*)(DecodeArgs);

template <typename T, int PPW, bool RUNS, bool ARGS> DecodeKernel pick_full(bool full) {
    return full ? decode_attn_mfma_kernel<T, PPW, RUNS, ARGS, true> : decode_attn_mfma_kernel<T, PPW, RUNS, ARGS, false>;
}
// Instances that launch_decode can reach: page lists in the arguments hold at
// most kArgPages pages, taken one or two per split; splits of more than two
// pages run them two at a time (one at a time for an odd count, so no run
// reads a page only to mask it out).  fp32 pages hold twice the K/V
// registers: runs of two would take 252 + 32 registers per lane and leave a
// SIMD one wave, so fp32 splits run one page at a time (32k positions: 30.0
// against 31.2 us per call; 64k: 52.7 against 55.0).
template <typename T> DecodeKernel pick_mfma(int ppw, bool args, bool full) {
    if (args) return ppw == 1 ? pick_full<T, 1, false, true>(full) : pick_full<T, 2, false, true>(full);
    switch (ppw) {
    case 1: return pick_full<T, 1, false, false>(full);
    case 2: return pick_full<T, 2, false, false>(full);
    default:
        if constexpr (sizeof(typename T::storage) == 2) {
            if (ppw % 2 == 0) return pick_full<T, 2, true, false>(full);
        }
        return pick_full<T, 1, true, false>(full);
    }
}

// Pages per split for `pages` cached pages (at most kMaxSplits splits).
// Measured at 1k-64k positions (fp16 cache, 4 kv heads): a page per split
// while there are at most 128 (4k positions: 64 workgroups per kv head), then
// two (fewer partials for the merge to read: 13.7 against 16.1 us per call at
// 16k), then 128 splits of runs.  The kernel holds 216 registers (VGPR +
// AGPR) per lane, so a SIMD runs two of its waves and the chip 512
// workgroups at once: 128 splits per kv head fill it in one round, where
// 2-page splits past 16k need a second (32k: 18.8 against 20.0 us per call;
// 64k, against 4-page splits issued at once at one wave per SIMD: 29.8
// against 38.2 us).
int decode_pages_per_split(int pages) {
    return pages <= 128 ? 1 : pages <= 256 ? 2 : (pages + 127) / 128;
}

hipError_t launch_decode(int kv_dtype, const DecodeArgs &args, hipStream_t s) {
    DecodeArgs a = args;
    // Work split: pages of the cached positions [0, L-1), the new token riding
    // with the last split.  One or two pages per split up to 16k positions,
    // all loads issued at once, then 128 splits whose pages are loaded in
    // runs of PPW (2, or 1 for an odd count); the split count stays within
    // kMaxSplits, the merge width.
    const int pages = (a.L - 1 + kPage - 1) / kPage;
    a.ppw = decode_pages_per_split(pages);
    a.nsplit = std::max(1, (pages + a.ppw - 1) / a.ppw);
    dim3 grid(a.nsplit, a.kv_heads), block(256);
    const bool in_args = a.pages_in_args != 0;
    if (in_args && a.ppw > 2) return hipErrorInvalidValue;
    const bool full = a.rope_dim == kHeadDim;
    DecodeKernel k;
    switch (kv_dtype) {
    case 0: k = pick_mfma<F32>(a.ppw, in_args, full); break;
    case 1: k = pick_mfma<F16>(a.ppw, in_args, full); break;
    case 2: k = pick_mfma<BF16>(a.ppw, in_args, full); break;
    default: return hipErrorInvalidValue;
    }
    {
        KernelSpan span("decode_attn", s, true);
        launch(span, k, grid, block, 0, s, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    const MergeArgs m{a.part_ml, a.part_acc, a.out, a.nsplit};
    const dim3 grid_m(a.kv_heads * kGroup, kHeadDim / 32);  // (q head, 32-dim quarter)
    KernelSpan span("decode_merge", s, true);
    if (a.nsplit <= 64)
        launch(span, decode_merge_kernel<2>, grid_m, dim3(256), 0, s, m);
    else if (a.nsplit <= 128)
        launch(span, decode_merge_kernel<4>, grid_m, dim3(256), 0, s, m);
    else
        launch(span, decode_merge_kernel<8>, grid_m, dim3(256), 0, s, m);
    return hipGetLastError();
}

}  // namespace hymt
