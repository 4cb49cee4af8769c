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
//   workgroup = (split, kv head), 4 waves, `ppw` 64-position pages per split.
//   Wave w owns positions [16w, 16w+16) of every page of its split and runs
//   its own online softmax over them: no workgroup barrier on the streaming
//   path.  A wave's 16 K rows and its 16x128 V^T sub-tile are each one
//   contiguous 4 KiB block; every load is a 16-byte vector.
//   The 4 wave partials are combined through LDS into one (m, l, acc[128])
//   per q head and split; splits are merged either by a second small kernel
//   or, with merge_inline, by the last workgroup of each kv head to finish
//   (device-coherent sc1 stores/loads and an atomic ticket; no cache flush).
#include "attn_kernels.hpp"
#include "device_common.hpp"

namespace hymt {

template <typename T> struct DecodeShape {
    static constexpr int D = kHeadDim, SUB = 16;
    static constexpr int VN = Vec16<T>::N;    // elements per 16-byte vector
    static constexpr int KCPR = D / VN;       // lanes per K row (16 or 32)
    static constexpr int KRPI = 64 / KCPR;    // K rows per wave load (4 or 2)
    static constexpr int KLD = SUB / KRPI;    // K loads per lane per sub-tile
    static constexpr int VCPD = SUB / VN;     // lanes per V^T row of a sub-tile (2 or 4)
    static constexpr int VDPI = 64 / VCPD;    // V^T rows per wave load (32 or 16)
    static constexpr int VLD = D / VDPI;      // V loads per lane per sub-tile
};

// Device-coherent (agent scope) accesses: sc1 on gfx950, visible across XCDs
// without writing back or invalidating whole L2 caches.
__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

// One 128-wide head row held as lanes (d, d+64): loads of x, rotation
// partners, cos/sin and gamma, all issued together (no dependent round trips).
struct RowIn {
    float x[2], xp[2], c[2], s[2], w[2];
    __device__ __forceinline__ void load(const float *row, const float *cs, const float *sn,
                                         const float *gamma, int lane, int half, int rope_dim) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int d = lane + 64 * e;
            x[e] = row[d];
            xp[e] = row[rope_partner(d, half, rope_dim)];
            const int i = rope_index(d, half, rope_dim);
            c[e] = cs[i];
            s[e] = sn[i];
            w[e] = gamma ? gamma[d] : 1.0f;
        }
    }
    // RoPE then RMSNorm (HunyuanDenseModel.Decode.cs:80-85): y = rope(x) * r * gamma
    __device__ __forceinline__ void finish(float *y, int lane, int half, int rope_dim, bool norm,
                                           float eps) const {
#pragma unroll
        for (int e = 0; e < 2; e++) y[e] = rope_elem(lane + 64 * e, x[e], xp[e], c[e], s[e], half, rope_dim);
        if (norm) {
            const float ss = group_sum<64>(y[0] * y[0] + y[1] * y[1]);
            const float r = 1.0f / sqrtf(ss / (float)kHeadDim + eps);
            y[0] = y[0] * r * w[0];
            y[1] = y[1] * r * w[1];
        }
    }
};

template <typename T, bool MULTI>
__global__ __launch_bounds__(256) void decode_attn_kernel(DecodeArgs a) {
    using Sh = DecodeShape<T>;
    constexpr int D = kHeadDim, G = kGroup, P = kPage, SUB = Sh::SUB;
    constexpr int VN = Sh::VN, KCPR = Sh::KCPR, KRPI = Sh::KRPI, KLD = Sh::KLD;
    constexpr int VCPD = Sh::VCPD, VDPI = Sh::VDPI, VLD = Sh::VLD;
    using S = typename T::storage;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Hkv = a.kv_heads;
    const int kvh = blockIdx.x % Hkv;
    const int split = blockIdx.x / Hkv;
    const int npages = (a.L + P - 1) / P;
    const int page0 = split * a.ppw;
    const int page_end = MULTI ? min(page0 + a.ppw, npages) : page0 + 1;
    const int newpos = a.L - 1;
    const bool owner = page_end == npages;

    __shared__ float s_q[G][D];
    __shared__ float s_knew[D], s_vnew[D];
    __shared__ float s_p[4][G][SUB];
    __shared__ float s_acc[4][G][D];
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_w[G][kMaxSplits];
    __shared__ float s_L[G];
    __shared__ uint32_t s_ticket;

    const size_t page_elems = (size_t)P * D;
    const S *kpool = (const S *)a.kpool;
    const S *vpool = (const S *)a.vpool;
    const int kc = lane % KCPR, kg = lane / KCPR;
    const int vc = lane % VCPD, vd = lane / VCPD;
    const int half = a.rope_half, rdim = a.rope_dim;

    // ---- prologue loads first: vmcnt retires in order, so the small q/k/v
    // rows must not queue behind the K/V stream ------------------------------
    RowIn qin, nin;
    qin.load(a.q + (size_t)(kvh * G + wave) * D, a.rope_cos, a.rope_sin, a.qnw, lane, half, rdim);
    if (owner && wave == 0)
        nin.load(a.knew + (size_t)kvh * D, a.rope_cos, a.rope_sin, a.knw, lane, half, rdim);
    if (owner && wave == 1)
        nin.load(a.vnew + (size_t)kvh * D, a.rope_cos, a.rope_sin, nullptr, lane, half, rdim);

    // this wave's sub-tile of page `page`: positions page*64 + 16*wave + [0, 16)
    uint4 kb[KLD], vb[VLD];
    auto load_sub = [&](int page, uint4 *kk, uint4 *vv) {
        const int base = page * P + SUB * wave;
        const int inmem = newpos - base;  // positions < newpos are resident
        const int phys = a.tab[page];
        const S *kp = kpool + ((size_t)phys * Hkv + kvh) * page_elems + (size_t)(SUB * wave) * D;
        const S *vp = vpool + ((size_t)phys * Hkv + kvh) * page_elems + (size_t)wave * D * SUB;
#pragma unroll
        for (int j = 0; j < KLD; j++) {
            const int r = kg + KRPI * j;
            kk[j] = r < inmem ? *(const uint4 *)(kp + (size_t)r * D + kc * VN) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < VLD; j++) {
            const int d = vd + VDPI * j;
            vv[j] = vc * VN < inmem ? *(const uint4 *)(vp + (size_t)d * SUB + vc * VN) : make_uint4(0, 0, 0, 0);
        }
    };
    load_sub(page0, kb, vb);

    // ---- prologue math: RoPE + RMSNorm of q (wave g: head g), new k and v ----
    {
        float y[2];
        qin.finish(y, lane, half, rdim, a.qnw != nullptr, a.eps);
        s_q[wave][lane] = y[0] * a.qscale;
        s_q[wave][lane + 64] = y[1] * a.qscale;
    }
    if (owner && wave < 2) {
        const int t = newpos % P;
        const int phys = a.tab[newpos / P];
        if (wave == 0) {
            float y[2];
            nin.finish(y, lane, half, rdim, a.knw != nullptr, a.eps);
            S *kp = (S *)kpool + ((size_t)phys * Hkv + kvh) * page_elems + (size_t)t * D;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const S st = to_elem<T>(y[e]);
                kp[lane + 64 * e] = st;
                s_knew[lane + 64 * e] = from_elem<T>(st);
            }
        } else {
            S *vp = (S *)vpool + ((size_t)phys * Hkv + kvh) * page_elems;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
                const S st = to_elem<T>(nin.x[e]);
                vp[v_off(t, d)] = st;
                s_vnew[d] = from_elem<T>(st);
            }
        }
    }
    __syncthreads();

    float qreg[G][VN];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < VN; e++) qreg[g][e] = s_q[g][kc * VN + e];

    float acc[VLD][G];
#pragma unroll
    for (int j = 0; j < VLD; j++)
#pragma unroll
        for (int g = 0; g < G; g++) acc[j][g] = 0.0f;
    float m_run[G], l_run[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m_run[g] = kFloor2;
        l_run[g] = 0.0f;
    }

    for (int page = page0; page < page_end; page++) {
        const int base = page * P + SUB * wave;
        const int nvalid = min(SUB, a.L - base);  // may be <= 0 past the end
        uint4 kn[KLD], vn[VLD];
        const bool more = MULTI && page + 1 < page_end;
        if (more) load_sub(page + 1, kn, vn);
        if (nvalid > 0) {
            // ---- scores of rows kg + KRPI*j --------------------------------
            float sc[KLD][G];
#pragma unroll
            for (int j = 0; j < KLD; j++) {
                const int r = kg + KRPI * j;
                float kv[VN];
                Vec16<T>::unpack(kb[j], kv);
                if (base + r == newpos) {
#pragma unroll
                    for (int e = 0; e < VN; e++) kv[e] = s_knew[kc * VN + e];
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    float s = 0.0f;
#pragma unroll
                    for (int e = 0; e < VN; e++) s = fmaf(qreg[g][e], kv[e], s);
                    sc[j][g] = lane_sum<KCPR>(s);
                }
            }
            // ---- online softmax over the sub-tile, per head ----------------
            float alpha[G];
#pragma unroll
            for (int g = 0; g < G; g++) {
                float mt = -INFINITY;
#pragma unroll
                for (int j = 0; j < KLD; j++)
                    if (kg + KRPI * j < nvalid) mt = fmaxf(mt, sc[j][g]);
#pragma unroll
                for (int o = KCPR; o < 64; o <<= 1) mt = fmaxf(mt, __shfl_xor(mt, o, 64));
                const float mnew = fmaxf(m_run[g], mt);
                alpha[g] = exp2f(m_run[g] - mnew);
                float ps = 0.0f;
#pragma unroll
                for (int j = 0; j < KLD; j++) {
                    const float p = kg + KRPI * j < nvalid ? exp2f(fmaxf(sc[j][g] - mnew, kFloor2)) : 0.0f;
                    sc[j][g] = p;
                    ps += p;
                }
#pragma unroll
                for (int o = KCPR; o < 64; o <<= 1) ps += __shfl_xor(ps, o, 64);
                l_run[g] = l_run[g] * alpha[g] + ps;
                m_run[g] = mnew;
            }
            if (kc == 0) {
#pragma unroll
                for (int j = 0; j < KLD; j++)
#pragma unroll
                    for (int g = 0; g < G; g++) s_p[wave][g][kg + KRPI * j] = sc[j][g];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

            // ---- P * V over the sub-tile: V^T rows vd + VDPI*j ---------------
            float preg[G][VN];
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < VN; e++) preg[g][e] = s_p[wave][g][vc * VN + e];
#pragma unroll
            for (int j = 0; j < VLD; j++) {
                const int d = vd + VDPI * j;
                float vv[VN];
                Vec16<T>::unpack(vb[j], vv);
#pragma unroll
                for (int e = 0; e < VN; e++) {
                    const int t = base + vc * VN + e;
                    if (t == newpos) vv[e] = s_vnew[d];
                    else if (t > newpos) vv[e] = 0.0f;
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    float s = acc[j][g] * alpha[g];
#pragma unroll
                    for (int e = 0; e < VN; e++) s = fmaf(preg[g][e], vv[e], s);
                    acc[j][g] = s;
                }
            }
            __builtin_amdgcn_wave_barrier();  // s_p is rewritten by the next sub-tile
        }
        if (more) {
#pragma unroll
            for (int j = 0; j < KLD; j++) kb[j] = kn[j];
#pragma unroll
            for (int j = 0; j < VLD; j++) vb[j] = vn[j];
        }
    }

    // ---- combine the 4 wave partials of this split --------------------------
#pragma unroll
    for (int j = 0; j < VLD; j++)
#pragma unroll
        for (int g = 0; g < G; g++) acc[j][g] = lane_sum<VCPD>(acc[j][g]);
    if (vc == 0) {
#pragma unroll
        for (int j = 0; j < VLD; j++)
#pragma unroll
            for (int g = 0; g < G; g++) s_acc[wave][g][vd + VDPI * j] = acc[j][g];
    }
    if (lane == 0) {  // m_run / l_run are uniform across the wave
#pragma unroll
        for (int g = 0; g < G; g++) {
            s_m[wave][g] = m_run[g];
            s_l[wave][g] = l_run[g];
        }
    }
    __syncthreads();

    const int g = tid >> 6, d0 = (tid & 63) * 2;  // thread -> head g, dims d0, d0+1
    const int h = kvh * G + g;
    float M = s_m[0][g];
#pragma unroll
    for (int w = 1; w < 4; w++) M = fmaxf(M, s_m[w][g]);
    float Lw = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float sc = exp2f(s_m[w][g] - M);
        Lw = fmaf(sc, s_l[w][g], Lw);
        o0 = fmaf(sc, s_acc[w][g][d0], o0);
        o1 = fmaf(sc, s_acc[w][g][d0 + 1], o1);
    }

    if (a.nsplit == 1) {
        const float inv = Lw > 0.0f ? 1.0f / Lw : 0.0f;
        *(float2 *)(a.out + (size_t)h * D + d0) = make_float2(o0 * inv, o1 * inv);
        return;
    }

    float *pacc = a.part_acc + ((size_t)h * kMaxSplits + split) * D + d0;
    float *pml = a.part_ml + ((size_t)h * kMaxSplits + split) * 2;
    if (!a.merge_inline) {
        *(float2 *)pacc = make_float2(o0, o1);
        if (d0 == 0) *(float2 *)pml = make_float2(M, Lw);
        return;
    }

    // ---- inline merge: the last split of this kv head combines all splits ---
    store_coherent(pacc, o0);
    store_coherent(pacc + 1, o1);
    if (d0 == 0) {
        store_coherent(pml, M);
        store_coherent(pml + 1, Lw);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are complete
    __syncthreads();
    if (tid == 0)
        s_ticket = __hip_atomic_fetch_add(&a.counters[kvh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_ticket != (uint32_t)(a.nsplit - 1)) return;

    {
        const float *ml = a.part_ml + (size_t)h * kMaxSplits * 2;
        float mloc = -INFINITY;
        for (int s = tid & 63; s < a.nsplit; s += 64) mloc = fmaxf(mloc, load_coherent(ml + 2 * s));
        const float Mg = group_max<64>(mloc);
        float lsum = 0.0f;
        for (int s = tid & 63; s < a.nsplit; s += 64) {
            const float w = exp2f(load_coherent(ml + 2 * s) - Mg);
            s_w[g][s] = w;
            lsum = fmaf(w, load_coherent(ml + 2 * s + 1), lsum);
        }
        lsum = group_sum<64>(lsum);
        if ((tid & 63) == 0) s_L[g] = lsum;
    }
    __syncthreads();
    {
        const float *pa = a.part_acc + (size_t)h * kMaxSplits * D + d0;
        float r0 = 0.0f, r1 = 0.0f;
        int s = 0;
        for (; s + 16 <= a.nsplit; s += 16) {
            float x0[16], x1[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                x0[i] = load_coherent(pa + (size_t)(s + i) * D);
                x1[i] = load_coherent(pa + (size_t)(s + i) * D + 1);
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                r0 = fmaf(s_w[g][s + i], x0[i], r0);
                r1 = fmaf(s_w[g][s + i], x1[i], r1);
            }
        }
        for (; s < a.nsplit; s++) {
            r0 = fmaf(s_w[g][s], load_coherent(pa + (size_t)s * D), r0);
            r1 = fmaf(s_w[g][s], load_coherent(pa + (size_t)s * D + 1), r1);
        }
        const float l = s_L[g];
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        *(float2 *)(a.out + (size_t)h * D + d0) = make_float2(r0 * inv, r1 * inv);
    }
    if (tid == 0) a.counters[kvh] = 0u;
}

// Merge of the split partials (second launch when merge_inline is off):
// block (head h, 32-dim slice); thread (split group sg of 8, dim).
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    constexpr int D = kHeadDim;
    const int h = blockIdx.x >> 2, dsl = (blockIdx.x & 3) * 32;
    const int tid = threadIdx.x, sg = tid >> 5, d = dsl + (tid & 31);
    __shared__ float s_w[kMaxSplits];
    __shared__ float s_part[8][32];
    __shared__ float s_L;
    const float *ml = a.part_ml + (size_t)h * kMaxSplits * 2;
    if (tid < 64) {
        float mloc = -INFINITY;
        for (int s = tid; s < a.nsplit; s += 64) mloc = fmaxf(mloc, ml[2 * s]);
        const float M = group_max<64>(mloc);
        float lsum = 0.0f;
        for (int s = tid; s < a.nsplit; s += 64) {
            const float w = exp2f(ml[2 * s] - M);
            s_w[s] = w;
            lsum = fmaf(w, ml[2 * s + 1], lsum);
        }
        lsum = group_sum<64>(lsum);
        if (tid == 0) s_L = lsum;
    }
    __syncthreads();
    const float *pa = a.part_acc + (size_t)h * kMaxSplits * D + d;
    float r = 0.0f;
#pragma unroll 4
    for (int s = sg; s < a.nsplit; s += 8) r = fmaf(s_w[s], pa[(size_t)s * D], r);
    s_part[sg][tid & 31] = r;
    __syncthreads();
    if (tid < 32) {
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) o += s_part[i][tid];
        const float l = s_L;
        a.out[(size_t)h * D + d] = l > 0.0f ? o / l : 0.0f;
    }
}

hipError_t launch_decode(int kv_dtype, const DecodeArgs &a, hipStream_t s) {
    dim3 grid(a.nsplit * a.kv_heads), block(256);
    const bool multi = a.ppw > 1;
    switch (kv_dtype * 2 + multi) {
    case 0: hipLaunchKernelGGL((decode_attn_kernel<F32, false>), grid, block, 0, s, a); break;
    case 1: hipLaunchKernelGGL((decode_attn_kernel<F32, true>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((decode_attn_kernel<F16, false>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((decode_attn_kernel<F16, true>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((decode_attn_kernel<BF16, false>), grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL((decode_attn_kernel<BF16, true>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1 || a.merge_inline) return e;
    hipLaunchKernelGGL(decode_merge_kernel, dim3(a.kv_heads * kGroup * 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hymt
