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
//   (one page per split until the split count reaches kMaxSplits, so a
//   4k-context layer spreads over 256 workgroups, every CU).
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
// are issued by load() before any use, in straight-line code, so they share
// one memory round trip and can be issued ahead of the K/V stream; finish()
// applies RoPE then RMSNorm (HunyuanDenseModel.Decode.cs:80-85).
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
        w[0] = gamma ? gamma[lane] : 1.0f;
        w[1] = gamma ? gamma[lane + 64] : 1.0f;
        if constexpr (FULL) {
            c[0] = c[1] = cosr[lane];
            s[0] = s[1] = sinr[lane];
        } else {
            // partner index d when d is not rotated; table index 0 then (the
            // table has at least one column whenever rdim > 0)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
#pragma unroll
                for (int r = 0; r < NR; r++) xp[r][e] = rows[r * kHeadDim + rope_partner(d, half, rdim)];
                c[e] = rdim > 0 ? cosr[rope_index(d, half, rdim)] : 1.0f;
                s[e] = rdim > 0 ? sinr[rope_index(d, half, rdim)] : 0.0f;
            }
        }
    }
    // Row r: RoPE (Ops.cs:157-165) then y = x * (1/sqrt(sum x^2/D + eps)) * gamma
    // (Ops.cs:62-88), times `scale`.
    __device__ __forceinline__ void finish(int r, float (&y)[2], int lane, int half, int rdim, bool norm,
                                           float eps, float scale) const {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float p = FULL ? x[r][1 - e] : xp[r][e];
            y[e] = FULL ? (e == 0 ? x[r][0] * c[0] - p * s[0] : p * s[1] + x[r][1] * c[1])
                        : rope_elem(lane + 64 * e, x[r][e], p, c[e], s[e], half, rdim);
        }
        if (norm) {
            const float ss = wave_sum64(y[0] * y[0] + y[1] * y[1]);
            const float rr = 1.0f / sqrtf(ss / (float)kHeadDim + eps);
            y[0] = y[0] * rr * w[0];
            y[1] = y[1] * rr * w[1];
        }
        y[0] *= scale;
        y[1] *= scale;
    }
};

// Decode for every cache type.
//   The cached positions [0, pos) are split by pages: workgroup (split, kv
//   head), 4 waves; wave w streams the 16-position sub-tile [16w, 16w+16) of
//   each of the split's pages.
//     S = K_sub . Qcat^T, lane (grp, c<4) gets head c at positions 4*grp + i
//     (its hi part; lanes c+4 hold the lo part).
//     O += Pcat . V_sub, lane (grp, c) gets rows 4*grp + i of dims 16*db + c,
//     rows 0-3 = hi(P) of the 4 heads, rows 4-7 = lo(P).
//   The new token (position pos) is one more position.  Wave 3 of the last
//   split computes it on the VALU from registers -- its K after RoPE + norm,
//   both rows rounded to the cache type as the reference reads them back from
//   its cache -- and adds it to the split's combine as a fifth partial; the
//   same wave appends the row to the cache at the end.  So no workgroup is
//   spent on a page that holds only the new token (L = 4097 runs exactly 256
//   workgroups), and no MFMA operand needs patching.
// PAGES_ARG: page ids come from the kernel arguments, else from the device
// page table; both are scalar loads issued first.
template <typename T, bool MULTI, bool PAGES_ARG, bool FULL>
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
    const int Hkv = a.kv_heads;
    const int split = blockIdx.x, kvh = blockIdx.y;  // grid (nsplit, kv heads)
    const int newpos = a.L - 1;                // cached positions [0, newpos)
    const int ncp = (newpos + P - 1) / P;      // cached pages
    // one page per split unless MULTI: the first page id's address then
    // depends on blockIdx alone and is loaded with the kernel arguments
    const int page0 = MULTI ? split * a.ppw : split;
    const int page_end = min(page0 + (MULTI ? a.ppw : 1), ncp);
    const bool last = split == a.nsplit - 1;
    const bool extra = last && wave == 3;      // the wave that adds the new token

    __shared__ __attribute__((aligned(16))) uint16_t s_qop[2][G][D];  // hi/lo q of the 4 heads
    __shared__ float s_qf[G][D];                                      // fp32 q, for the new token
    __shared__ __attribute__((aligned(16))) float s_o[4][2][D][G];       // per wave: hi/lo rows
    __shared__ __attribute__((aligned(16))) float s_xo[D][G];            // the new token
    __shared__ float s_m[5][G], s_l[5][G];                                // [4]: the new token

    const size_t page_elems = (size_t)P * D;
    const S *kpool = (const S *)a.kpool;
    const S *vpool = (const S *)a.vpool;
    const int half = a.rope_half, rdim = a.rope_dim;

    // ---- 1. page ids: the K/V addresses hang on them -----------------------
    // Loads are never skipped by a branch: after a conditional block of loads
    // the wait counts must cover the path without them, which makes every
    // later wait drain the K/V stream.  Look-ahead pages past the split clamp
    // to its last page (a re-read from L2); with no cached page (pos = 0) the
    // page of pos is read and ignored.
    auto page_id = [&](int p) { return PAGES_ARG ? a.pages[p] : a.tab[p]; };
    const int plast = max(page_end - 1, page0);
    const int phys0 = page_id(page0);
    const int phys1 = MULTI ? page_id(min(page0 + 1, plast)) : 0;

    // ---- 2. q rows and the new k, v rows ------------------------------------
    // vmcnt retires in order: these small rows are issued ahead of the K/V
    // stream so the q operand is built while it is in flight.  Wave w loads
    // q head w of the group; every wave loads the new rows (1.5 KiB, cached)
    // so that all loads sit in one straight-line block.
    RowsIn<1, FULL> qin;
    RowsIn<1, FULL> kin;
    qin.load(a.q + (size_t)(kvh * G + wave) * D, a.rope_cos, a.rope_sin, a.qnw, lane, half, rdim);
    kin.load(a.knew + (size_t)kvh * D, a.rope_cos, a.rope_sin, a.knw, lane, half, rdim);
    const float vnew0 = a.vnew[(size_t)kvh * D + lane];
    const float vnew1 = a.vnew[(size_t)kvh * D + lane + 64];

    // ---- 3. the K/V stream --------------------------------------------------
    // f16/bf16 pages: wave w takes the 16 positions of V chunks 2w and 2w+1,
    // so that its V loads are whole 16-byte chunks; S row / P.V index
    // 4 grp + i of the wave is page position posw(i) below.
    // K A-operand: lane (grp, c) = K row c (position posw of index c), dims
    //   32*ks + 8*grp + [0, 8): two 128-byte segments per 16 lanes.
    // V B-operand: lane (grp, c) = V^T row 16*db + c, indices 4*grp + [0, 4):
    //   half (grp & 1) of V chunk (2 w + (grp >> 1), 16 db + c).
    // Whole sub-tiles are loaded (pages are fully allocated); rows at or past
    // pos are masked out of the scores and zeroed in V before use.
    //   f32 pages (row-major K, V^T sub-tiles): the same operands as fp32,
    //   two 16-byte K loads per ks and one 16-byte V load per db.
    constexpr int KL = W4 ? 8 : 4;
    using VL = typename std::conditional<W4, uint4, uint2>::type;
    uint4 ka[KL], kn[KL];
    VL vb[8], vn[8];
    auto load_sub = [&](int phys, uint4 *kk, VL *vv) {
        const size_t pb = ((size_t)phys * Hkv + kvh) * page_elems;
        if constexpr (W4) {
            const S *kp = kpool + pb + (size_t)(SUB * wave + c) * D + 8 * grp;
            const S *vp = vpool + pb + (size_t)(wave * D + c) * SUB + 4 * grp;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                kk[2 * ks] = *(const uint4 *)(kp + 32 * ks);
                kk[2 * ks + 1] = *(const uint4 *)(kp + 32 * ks + 4);
            }
#pragma unroll
            for (int db = 0; db < 8; db++) vv[db] = *(const VL *)(vp + 256 * db);
        } else {
            const S *kp = kpool + pb + 2048 * (2 * (wave >> 1) + ((c >> 2) & 1)) + 128 * grp +
                          8 * (8 * (wave & 1) + 4 * (c >> 3) + (c & 3));
            const S *vp = vpool + pb + (size_t)(2 * wave + (grp >> 1)) * 1024 + 8 * c + 4 * (grp & 1);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) kk[ks] = *(const uint4 *)(kp + 512 * ks);
#pragma unroll
            for (int db = 0; db < 8; db++) vv[db] = *(const VL *)(vp + 128 * db);
        }
    };
    load_sub(phys0, ka, vb);
    if (MULTI) load_sub(phys1, kn, vn);  // two pages in flight

    // ---- 4. q operand: wave w applies RoPE + norm to head w and stores its
    // hi/lo split (and the fp32 row) in LDS; one barrier shares the 4 heads --
    {
        float y[2];
        qin.finish(0, y, lane, half, rdim, a.qnw != nullptr, a.eps, a.qscale);
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const uint32_t pr = split_pair<Op>(y[e]);
            s_qop[0][wave][lane + 64 * e] = (uint16_t)pr;
            s_qop[1][wave][lane + 64 * e] = (uint16_t)(pr >> 16);
            s_qf[wave][lane + 64 * e] = y[e];
        }
    }
    __syncthreads();
    // Qcat B-operand: lane (grp, c), dims 32*ks + 8*grp + [0, 8):
    // c < 4 -> hi(q_c), 4 <= c < 8 -> lo(q_{c-4}), else 0
    uint4 qb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
        qb[ks] = c < 8 ? *(const uint4 *)&s_qop[c >> 2][c & 3][32 * ks + 8 * grp] : make_uint4(0, 0, 0, 0);

    // ---- 5. the new token: K after RoPE + norm and V, rounded to the cache
    // type (Ops.ConvertToBf16, Ops.cs:658-680), then its weight for each head
    // in the softmax's base-2 units: m = max(s, floor), l = exp2(max(s-m, floor)).
    // Its cache stores are issued at the end: vmcnt retires in order, so
    // stores issued here would hold up every later wait on the K/V stream.
    S knew_st[2] = {}, vnew_st[2] = {};
    if (extra) {
        float ky[2];
        kin.finish(0, ky, lane, half, rdim, a.knw != nullptr, a.eps, 1.0f);
        knew_st[0] = to_elem<T>(ky[0]);
        knew_st[1] = to_elem<T>(ky[1]);
        vnew_st[0] = to_elem<T>(vnew0);
        vnew_st[1] = to_elem<T>(vnew1);
        const float k0 = from_elem<T>(knew_st[0]), k1 = from_elem<T>(knew_st[1]);
        const float v0 = from_elem<T>(vnew_st[0]), v1 = from_elem<T>(vnew_st[1]);
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float sc = wave_sum64(s_qf[g][lane] * k0 + s_qf[g][lane + 64] * k1);
            const float m = fmaxf(sc, kFloor2);
            const float l = exp2f(fmaxf(sc - m, kFloor2));
            s_xo[lane][g] = l * v0;
            s_xo[lane + 64][g] = l * v1;
            if (lane == 0) {
                s_m[4][g] = m;
                s_l[4][g] = l;
            }
        }
    }

    // ---- 6. attention over the split's cached sub-tiles ---------------------
    // page position of S row / P.V index 4 grp + i of this wave, and the
    // smallest one (f32 pages: the sub-tile [16 w, 16 w + 16))
    auto posw = [&](int i) {
        return W4 ? SUB * wave + 4 * grp + i
                  : 32 * (wave >> 1) + 8 * (wave & 1) + 4 * (grp >> 1) + 16 * (grp & 1) + i;
    };
    const int pmin = W4 ? SUB * wave : 32 * (wave >> 1) + 8 * (wave & 1);
    f32x4 acc[8];
#pragma unroll
    for (int db = 0; db < 8; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kFloor2, l_run = 0.0f;  // lanes c < 4: head c

    for (int page = page0; page < page_end; page++) {
        const int nv = newpos - page * P;  // positions of this page below pos
        if (nv > pmin) {
            // scores: lane (grp, c<4) <- head c, positions 4*grp + i
            f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                if constexpr (W4) {
                    uint4 hi, lo;
                    split8(ka[2 * ks], ka[2 * ks + 1], hi, lo);
                    sacc = M::qk(hi, qb[ks], sacc);
                    sacc = M::qk(lo, qb[ks], sacc);
                } else {
                    sacc = M::qk(ka[ks], qb[ks], sacc);
                }
            }
            float sc[4], mt = kFloor2;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[i] = sacc[i] + dpp_from_plus4(sacc[i]);
                if (posw(i) < nv) mt = fmaxf(mt, sc[i]);
            }
            mt = xrow32_max(xrow16_max(mt));
            const float mnew = fmaxf(m_run, mt);
            float p[4], ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[i] = posw(i) < nv ? exp2f(fmaxf(sc[i] - mnew, kFloor2)) : 0.0f;
                ps += p[i];
            }
            ps = xrow32_sum(xrow16_sum(ps));
            // Pcat A-operand: lane (grp, r): r<4 hi(p_r), 4<=r<8 lo(p_{r-4})
            uint32_t hp[2], lp[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t p0 = split_pair<Op>(p[2 * e]), p1 = split_pair<Op>(p[2 * e + 1]);
                hp[e] = (p0 & 0xFFFFu) | (p1 << 16);
                lp[e] = dpp_from_minus4((p0 >> 16) | (p1 & 0xFFFF0000u));
            }
            const uint2 pa = c < 4 ? make_uint2(hp[0], hp[1]) : c < 8 ? make_uint2(lp[0], lp[1]) : make_uint2(0u, 0u);
            if (MULTI) {  // rescale the running sums (a single sub-tile starts from zero)
                const float alpha = exp2f(m_run - mnew);
                l_run = l_run * alpha + ps;
                float al[4];
#pragma unroll
                for (int i = 0; i < 4; i++) al[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), i));  // head i
#pragma unroll
                for (int db = 0; db < 8; db++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[db][i] *= al[i];
            } else {
                l_run = ps;
            }
            m_run = mnew;
            // V: zero the positions at or past pos (halfword masks of this
            // lane's 4 positions); they may hold stale data
            uint32_t keep[2] = {0xFFFFFFFFu, 0xFFFFFFFFu};
            if (nv < P) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (posw(j) >= nv) keep[j >> 1] &= ~(0xFFFFu << (16 * (j & 1)));
            }
            if constexpr (W4) {
#pragma unroll
                for (int db = 0; db < 8; db++) {
                    uint2 hi, lo;
                    split4(vb[db], keep, hi, lo);
                    acc[db] = M::pv(pa, hi, acc[db]);
                    acc[db] = M::pv(pa, lo, acc[db]);
                }
            } else {
#pragma unroll
                for (int db = 0; db < 8; db++)
                    acc[db] = M::pv(pa, make_uint2(vb[db].x & keep[0], vb[db].y & keep[1]), acc[db]);
            }
        }
        if (MULTI) {
#pragma unroll
            for (int ks = 0; ks < KL; ks++) ka[ks] = kn[ks];
#pragma unroll
            for (int db = 0; db < 8; db++) vb[db] = vn[db];
            load_sub(page_id(min(page + 2, plast)), kn, vn);
        }
    }

    // ---- 7. combine the wave partials (and the new token) ------------------
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
            if (a.nsplit == 1) {
                a.out[(size_t)h * D + d] = Lx[j] > 0.0f ? O[j] / Lx[j] : 0.0f;
            } else {
                a.part_acc[((size_t)h * kMaxSplits + split) * D + d] = O[j];
                if (d == 0) *(float2 *)(a.part_ml + ((size_t)h * kMaxSplits + split) * 2) = make_float2(Mx[j], Lx[j]);
            }
        }
    }
    // ---- 8. append the new row to the cache ---------------------------------
    if (extra) {
        const int phys = page_id(newpos / P), t = newpos % P;
        S *kp = (S *)kpool + ((size_t)phys * Hkv + kvh) * page_elems;
        S *vp = (S *)vpool + ((size_t)phys * Hkv + kvh) * page_elems;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            kp[k_off<sizeof(S)>(t, lane + 64 * e)] = knew_st[e];
            vp[v_off<sizeof(S)>(t, lane + 64 * e)] = vnew_st[e];
        }
    }
}

// Merge of the split partials (the second launch of a multi-split call):
// out[h] = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s, M = max_s m_s.
// Workgroup = q head; thread = (split group sg of 8, 4 dims).  Every thread
// issues all its loads (float2 (m, l) and float4 acc per split) at once; the
// 8 split groups are combined through LDS.
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    constexpr int D = kHeadDim, NG = 8, PER = kMaxSplits / NG;
    const int h = blockIdx.x, d4 = threadIdx.x & 31, sg = threadIdx.x >> 5;
    __shared__ float s_m[NG], s_l[NG];
    __shared__ float4 s_o[NG][32];
    const float2 *ml = (const float2 *)(a.part_ml + (size_t)h * kMaxSplits * 2);
    const float4 *pa = (const float4 *)(a.part_acc + (size_t)h * kMaxSplits * D) + d4;
    float2 mlv[PER];
    float4 x[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int s = sg + NG * k;
        const bool ok = s < a.nsplit;
        mlv[k] = ok ? ml[s] : make_float2(-INFINITY, 0.0f);
        x[k] = ok ? pa[(size_t)s * (D / 4)] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; k++) M = fmaxf(M, mlv[k].x);
    float L = 0.0f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    if (M != -INFINITY) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const float w = exp2f(mlv[k].x - M);
            L = fmaf(w, mlv[k].y, L);
            O.x = fmaf(w, x[k].x, O.x);
            O.y = fmaf(w, x[k].y, O.y);
            O.z = fmaf(w, x[k].z, O.z);
            O.w = fmaf(w, x[k].w, O.w);
        }
    }
    if (d4 == 0) {
        s_m[sg] = M;
        s_l[sg] = L;
    }
    s_o[sg][d4] = O;
    __syncthreads();
    if (sg == 0) {
        float Mt = s_m[0];
#pragma unroll
        for (int g = 1; g < NG; g++) Mt = fmaxf(Mt, s_m[g]);
        float Lt = 0.0f;
        float4 Ot = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int g = 0; g < NG; g++) {
            if (s_m[g] == -INFINITY) continue;
            const float w = exp2f(s_m[g] - Mt);
            const float4 o = s_o[g][d4];
            Lt = fmaf(w, s_l[g], Lt);
            Ot.x = fmaf(w, o.x, Ot.x);
            Ot.y = fmaf(w, o.y, Ot.y);
            Ot.z = fmaf(w, o.z, Ot.z);
            Ot.w = fmaf(w, o.w, Ot.w);
        }
        const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
        ((float4 *)(a.out + (size_t)h * D))[d4] = make_float4(Ot.x * inv, Ot.y * inv, Ot.z * inv, Ot.w * inv);
    }
}

// ---- the decode workspace of hymt_attn_decode_noalloc ------------------------
// A file-scope device array holds the split partials -- (m, l) then acc, laid
// out as DecodeArgs.part_ml / part_acc for up to kScratchHeads q heads -- so
// that a decode call needs no device allocation.  Every GPU that loads the
// library holds its own copy until the process ends; its address on a
// device comes from hipGetSymbolAddress with that device current (in host
// code the array's name is not a device address).  Every call on one GPU
// shares the array: the splits overwrite every partial the merge reads, so
// nothing needs clearing, and calls that overlap on one GPU race.
constexpr int kScratchHeads = 32;
constexpr size_t kScratchMl = (size_t)kScratchHeads * kMaxSplits * 2;        // floats
constexpr size_t kScratchAcc = (size_t)kScratchHeads * kMaxSplits * kHeadDim;  // floats
static __device__ __align__(256) float scratch[kScratchMl + kScratchAcc];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch[kScratchDevices] = {};
}  // namespace

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

template <typename T> DecodeKernel pick_mfma(bool multi, bool args, bool full) {
    const int i = multi * 4 + args * 2 + full;
    static const DecodeKernel k[8] = {
        decode_attn_mfma_kernel<T, false, false, false>, decode_attn_mfma_kernel<T, false, false, true>,
        decode_attn_mfma_kernel<T, false, true, false>,  decode_attn_mfma_kernel<T, false, true, true>,
        decode_attn_mfma_kernel<T, true, false, false>,  decode_attn_mfma_kernel<T, true, false, true>,
        decode_attn_mfma_kernel<T, true, true, false>,   decode_attn_mfma_kernel<T, true, true, true>};
    return k[i];
}

hipError_t launch_decode(int kv_dtype, const DecodeArgs &args, hipStream_t s) {
    DecodeArgs a = args;
    // Work split: pages of the cached positions [0, L-1), the new token riding
    // with the last split.  One page per split until the split count reaches
    // kMaxSplits (the merge width).
    const int pages = (a.L - 1 + kPage - 1) / kPage;
    a.ppw = std::max(1, (pages + kMaxSplits - 1) / kMaxSplits);
    a.nsplit = std::max(1, (pages + a.ppw - 1) / a.ppw);
    dim3 grid(a.nsplit, a.kv_heads), block(256);
    const bool multi = a.ppw > 1, in_args = a.pages_in_args != 0;
    const bool full = a.rope_dim == kHeadDim;
    DecodeKernel k;
    switch (kv_dtype) {
    case 0: k = pick_mfma<F32>(multi, in_args, full); break;
    case 1: k = pick_mfma<F16>(multi, in_args, full); break;
    case 2: k = pick_mfma<BF16>(multi, in_args, full); break;
    default: return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(k, grid, block, 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    hipLaunchKernelGGL(decode_merge_kernel, dim3(a.kv_heads * kGroup), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hymt
