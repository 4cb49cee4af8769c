// prefill_attn.hip -- causal GQA prefill attention for gfx950.
//
// Replaces the prefill attention of HunyuanDenseModel.PrefillAttention
// (HunyuanDenseModel.Prefill.cs:53-83): RoPE + Q/K RMSNorm + append of the
// chunk's K/V, then AttentionScores -> SoftmaxCausal -> AttentionCombine
// (Ops.cs:198-221, 359-455, 535-595), as the Vulkan pf_kvprep + pf_fa32 pair
// does on other GPUs (pf_kvprep.comp, pf_fa32.comp).
//
// Three kernels:
//  prefill_prep   one workgroup per token: RoPE/norm q and k, write k and v
//                 into the paged cache (cache dtype), write q in the MFMA
//                 operand type pre-scaled by log2(e)/sqrt(D).
//  prefill_flash  one workgroup per (kv head, 32-row q block, kv tile range):
//                 4 waves = the 4 q heads of the GQA group sharing every
//                 K/V tile staged in LDS.  S^T = K Q^T and O^T += V^T P^T on
//                 v_mfma_f32_16x16x32_{bf16,f16}, single-pass online
//                 softmax in base 2 with the reference's -80 floor.
//  prefill_merge  combines the (m, l, O) partials of q blocks whose kv range
//                 was split over several workgroups (long cached prefixes).
#include "attn_kernels.hpp"
#include "device_common.hpp"

namespace hymt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ prep
template <typename T>
__global__ __launch_bounds__(256) void prefill_prep_kernel(PrepArgs a) {
    constexpr int D = kHeadDim, P = kPage;
    using S = typename T::storage;
    const int m = blockIdx.x;
    const int pos = a.pos0 + m;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int Hq = a.heads, Hkv = a.kv_heads;
    const float *cs = a.rope_cos + (size_t)pos * a.rope_half;
    const float *sn = a.rope_sin + (size_t)pos * a.rope_half;
    const int phys = a.tab[pos / P], t = pos % P;

    auto load = [&](const void *base, size_t i) -> float {
        return a.io_bf16 ? bf16_to_f32(((const uint16_t *)base)[i]) : ((const float *)base)[i];
    };

    for (int row = wave; row < Hq + 2 * Hkv; row += 4) {
        if (row < Hq + Hkv) {
            const bool isq = row < Hq;
            const int h = isq ? row : row - Hq;
            const void *src = isq ? a.q : a.k;
            const size_t off = (size_t)m * (isq ? Hq : Hkv) * D + (size_t)h * D;
            float y[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
                const float x = load(src, off + d);
                if (d < a.rope_half) {
                    y[e] = x * cs[d] - load(src, off + d + a.rope_half) * sn[d];
                } else if (d < a.rope_dim) {
                    const int i = d - a.rope_half;
                    y[e] = load(src, off + i) * sn[i] + x * cs[i];
                } else {
                    y[e] = x;
                }
            }
            const float *w = isq ? a.qnw : a.knw;
            if (w) {
                float ss = group_sum<64>(y[0] * y[0] + y[1] * y[1]);
                float r = 1.0f / sqrtf(ss / (float)D + a.eps);
                y[0] = y[0] * r * w[lane];
                y[1] = y[1] * r * w[lane + 64];
            }
            if (isq) {
                S *qp = (S *)a.qp + ((size_t)h * a.seq_pad + m) * D;
                qp[lane] = to_elem<T>(y[0] * a.qscale);
                qp[lane + 64] = to_elem<T>(y[1] * a.qscale);
            } else {
                S *kp = (S *)a.kpool + ((size_t)phys * Hkv + h) * (size_t)(P * D) + (size_t)t * D;
                kp[lane] = to_elem<T>(y[0]);
                kp[lane + 64] = to_elem<T>(y[1]);
            }
        } else {
            const int h = row - Hq - Hkv;
            const size_t off = (size_t)m * Hkv * D + (size_t)h * D;
            S *vp = (S *)a.vpool + ((size_t)phys * Hkv + h) * (size_t)(P * D);
            vp[v_off(t, lane)] = to_elem<T>(load(a.v, off + lane));
            vp[v_off(t, lane + 64)] = to_elem<T>(load(a.v, off + lane + 64));
        }
    }
}

hipError_t launch_prefill_prep(int kv_dtype, const PrepArgs &a, hipStream_t s) {
    dim3 grid(a.seq), block(256);
    switch (kv_dtype) {
    case 1: hipLaunchKernelGGL(prefill_prep_kernel<F16>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(prefill_prep_kernel<BF16>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ work items
// Items are enumerated heaviest q block first; a q block with more than
// `cap` kv tiles is split into ceil(tiles/cap) consecutive items.
__host__ __device__ inline int flash_splits(int tiles, int cap) { return (tiles + cap - 1) / cap; }

struct FlashItem {
    int qb, split, nsplit, t0, t1, first;  // `first`: item index of split 0
};

__device__ inline FlashItem flash_item(const FlashArgs &a, int item) {
    FlashItem it;
    int first = 0;
    for (int qb = a.nqb - 1; qb >= 0; qb--) {
        const int nt = flash_tiles(a.pos0, qb, a.seq);
        const int ns = flash_splits(nt, a.cap);
        if (item < first + ns) {
            const int s = item - first;
            it.qb = qb;
            it.split = s;
            it.nsplit = ns;
            it.t0 = s * nt / ns;
            it.t1 = (s + 1) * nt / ns;
            it.first = first;
            return it;
        }
        first += ns;
    }
    it.qb = -1;
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

// K tile rows live at LDS row swz(r): bits 2 and 4 of the row index swapped,
// so the 16 rows one quarter-wave reads for an S^T block hit distinct banks.
__device__ __forceinline__ int kswz(int r) { return (r & ~0x14) | ((r & 4) << 2) | ((r & 16) >> 2); }

// Kv row of S^T block kb, block row r.  Chosen so that, after the softmax,
// lane (grp, c) holds P for positions 32*(kb/2) + 8*grp + [0, 8) of both
// blocks of a pair: the P^T operand then pairs with 8 consecutive positions
// of a V^T row.
__device__ __forceinline__ int krow(int kb, int r) {
    return 32 * (kb >> 1) + 8 * (r >> 2) + 4 * (kb & 1) + (r & 3);
}

template <typename T>
__global__ __launch_bounds__(256) void prefill_flash_kernel(FlashArgs a) {
    constexpr int D = kHeadDim, P = kPage, G = kGroup;
    constexpr int KLD = D + 8;  // 272-byte K rows
    constexpr int VLD = P + 8;  // 144-byte V^T rows
    typedef typename Mfma<T>::vec vec;
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][P * KLD];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][D * VLD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
    const int h = kvh * G + wave;
    const int q0 = it.qb * 32;

    // q fragments: B operand of S^T = K Q^T, lane (grp, c) -> row c, dims 8*grp..
    vec qf[2][4];
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
        const int row = q0 + qq * 16 + c;
        const uint16_t *qr = (const uint16_t *)a.qp + ((size_t)h * a.seq_pad + row) * D;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            uint4 u = row < a.seq ? *(const uint4 *)(qr + ks * 32 + grp * 8) : make_uint4(0, 0, 0, 0);
            qf[qq][ks] = __builtin_bit_cast(vec, u);
        }
    }

    f32x4 o[8][2];
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int qq = 0; qq < 2; qq++) o[db][qq] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrun[2] = {kFloor2, kFloor2}, lrun[2] = {0.f, 0.f};

    const int L = a.pos0 + a.seq;
    const size_t page_elems = (size_t)P * D;
    const uint16_t *kpool = (const uint16_t *)a.kpool;
    const uint16_t *vpool = (const uint16_t *)a.vpool;

    uint4 rk[4], rv[4];
    auto fetch = [&](int tile) {
        const int phys = a.tab[tile];
        const uint16_t *kp = kpool + ((size_t)phys * Hkv + kvh) * page_elems;
        const uint16_t *vp = vpool + ((size_t)phys * Hkv + kvh) * page_elems;
        const int nvalid = L - tile * P;  // positions >= L hold no data
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int idx = tid + 256 * j;
            rk[j] = *(const uint4 *)(kp + (size_t)idx * 8);
            uint4 v = *(const uint4 *)(vp + (size_t)idx * 8);
            // idx -> sub-tile idx/256, d (idx%256)/2, positions 16*sub + 8*(idx%2) + [0,8)
            const int col0 = (idx / 256) * 16 + (idx % 2) * 8;
            if (col0 + 8 > nvalid) {  // zero V^T entries of unwritten positions
                uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (col0 + 2 * e >= nvalid) w[e] &= 0xFFFF0000u;
                    if (col0 + 2 * e + 1 >= nvalid) w[e] &= 0x0000FFFFu;
                }
                v = make_uint4(w[0], w[1], w[2], w[3]);
            }
            rv[j] = v;
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int idx = tid + 256 * j;
            const int kr = idx / 16, kc = idx % 16;
            *(uint4 *)(&sK[buf][kswz(kr) * KLD + kc * 8]) = rk[j];
            const int vr = (idx % 256) / 2, vcol = (idx / 256) * 16 + (idx % 2) * 8;
            *(uint4 *)(&sV[buf][vr * VLD + vcol]) = rv[j];
        }
    };

    fetch(it.t0);
    stash(0);
    __syncthreads();

    for (int t = it.t0; t < it.t1; t++) {
        const int buf = (t - it.t0) & 1;
        const bool more = t + 1 < it.t1;
        if (more) fetch(t + 1);

        // ---- S^T = K Q^T (64 kv x 32 q) ----
        f32x4 sacc[4][2];
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int qq = 0; qq < 2; qq++) sacc[kb][qq] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const int r = kswz(krow(kb, c));
                vec kf = __builtin_bit_cast(vec, *(const uint4 *)(&sK[buf][r * KLD + ks * 32 + grp * 8]));
#pragma unroll
                for (int qq = 0; qq < 2; qq++) sacc[kb][qq] = Mfma<T>::mma(kf, qf[qq][ks], sacc[kb][qq]);
            }
        }

        // ---- causal mask + online softmax (column c = q row) ----
        const int kvbase = t * P;
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int qpos = a.pos0 + q0 + qq * 16 + c;
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int kv = kvbase + krow(kb, grp * 4 + i);
                    if (kv <= qpos) mx = fmaxf(mx, sacc[kb][qq][i]);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(mrun[qq], mx);
            const float alpha = exp2f(mrun[qq] - mnew);
            float ps = 0.f;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int kv = kvbase + krow(kb, grp * 4 + i);
                    const float p = kv <= qpos ? exp2f(fmaxf(sacc[kb][qq][i] - mnew, kFloor2)) : 0.f;
                    sacc[kb][qq][i] = p;
                    ps += p;
                }
            lrun[qq] = lrun[qq] * alpha + ps;
            mrun[qq] = mnew;
#pragma unroll
            for (int db = 0; db < 8; db++) o[db][qq] *= alpha;
        }

        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ks2++) {
            vec pf[2];
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                uint16_t e[8];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    e[i] = to_elem<T>(sacc[2 * ks2][qq][i]);
                    e[4 + i] = to_elem<T>(sacc[2 * ks2 + 1][qq][i]);
                }
                uint4 u = make_uint4(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                                     e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16));
                pf[qq] = __builtin_bit_cast(vec, u);
            }
#pragma unroll
            for (int db = 0; db < 8; db++) {
                vec vf = __builtin_bit_cast(vec, *(const uint4 *)(&sV[buf][(db * 16 + c) * VLD + ks2 * 32 + grp * 8]));
#pragma unroll
                for (int qq = 0; qq < 2; qq++) o[db][qq] = Mfma<T>::mma(vf, pf[qq], o[db][qq]);
            }
        }

        if (more) stash(buf ^ 1);
        __syncthreads();
    }

    // ---- finish: row sums across the 4 lane groups ----
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
        float l = lrun[qq];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        lrun[qq] = l;
    }
    const int qdim = a.heads * D;
    if (it.nsplit == 1) {
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int row = q0 + qq * 16 + c;
            if (row >= a.seq) continue;
            const float inv = lrun[qq] > 0.f ? 1.0f / lrun[qq] : 0.f;
            float *orow = a.out + (size_t)row * qdim + (size_t)h * D + grp * 4;
#pragma unroll
            for (int db = 0; db < 8; db++) {
                f32x4 v = o[db][qq] * inv;
                *(float4 *)(orow + db * 16) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    } else {
        const size_t slot = (size_t)kvh * a.items_per_kvh + item_idx;
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int r = qq * 16 + c;
            float *po = a.part_o + ((slot * G + wave) * 32 + r) * D + grp * 4;
#pragma unroll
            for (int db = 0; db < 8; db++) {
                f32x4 v = o[db][qq];
                *(float4 *)(po + db * 16) = make_float4(v[0], v[1], v[2], v[3]);
            }
            if (grp == 0) {
                float *pm = a.part_ml + ((slot * G + wave) * 32 + r) * 2;
                pm[0] = mrun[qq];
                pm[1] = lrun[qq];
            }
        }
    }
}

hipError_t launch_prefill_flash(int kv_dtype, const FlashArgs &a, int total_items, hipStream_t s) {
    (void)total_items;
    const int R = 8 / a.kv_heads;
    const int per_xcd = (a.items_per_kvh + R - 1) / R;
    dim3 grid(per_xcd * 8), block(256);
    switch (kv_dtype) {
    case 1: hipLaunchKernelGGL(prefill_flash_kernel<F16>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(prefill_flash_kernel<BF16>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ merge
__global__ __launch_bounds__(256) void prefill_merge_kernel(FlashArgs a) {
    constexpr int D = kHeadDim, G = kGroup;
    const int kvh = blockIdx.x % a.kv_heads;
    const int qb = blockIdx.x / a.kv_heads;
    // locate q block qb's items
    int first = 0, ns = 0;
    for (int b = a.nqb - 1; b >= 0; b--) {
        const int n = flash_splits(flash_tiles(a.pos0, b, a.seq), a.cap);
        if (b == qb) { ns = n; break; }
        first += n;
    }
    if (ns <= 1) return;
    const int qdim = a.heads * D;
    const int d = threadIdx.x % D;
    for (int rr = threadIdx.x / D; rr < G * 32; rr += 256 / D) {
        const int g = rr / 32, r = rr % 32;
        const int row = qb * 32 + r;
        if (row >= a.seq) continue;
        float M = -INFINITY;
        for (int s = 0; s < ns; s++) {
            const size_t slot = (size_t)kvh * a.items_per_kvh + first + s;
            M = fmaxf(M, a.part_ml[((slot * G + g) * 32 + r) * 2]);
        }
        float Ls = 0.f, acc = 0.f;
        for (int s = 0; s < ns; s++) {
            const size_t slot = (size_t)kvh * a.items_per_kvh + first + s;
            const float *pm = a.part_ml + ((slot * G + g) * 32 + r) * 2;
            const float w = exp2f(pm[0] - M);
            Ls += w * pm[1];
            acc = fmaf(w, a.part_o[((slot * G + g) * 32 + r) * D + d], acc);
        }
        a.out[(size_t)row * qdim + (size_t)(kvh * G + g) * D + d] = Ls > 0.f ? acc / Ls : 0.f;
    }
}

hipError_t launch_prefill_merge(const FlashArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(prefill_merge_kernel, dim3(a.nqb * a.kv_heads), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hymt
