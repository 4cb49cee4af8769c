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

typedef float f32x4 __attribute__((ext_vector_type(4)));

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
        x[0] = row[lane];
        x[1] = row[lane + 64];
        w[0] = gamma ? gamma[lane] : 1.0f;
        w[1] = gamma ? gamma[lane + 64] : 1.0f;
        if (half == 64) {  // full-width NeoX RoPE: the partner of d is d^64, same lane
            xp[0] = x[1];
            xp[1] = x[0];
            c[0] = c[1] = cs[lane];
            s[0] = s[1] = sn[lane];
            return;
        }
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int d = lane + 64 * e;
            xp[e] = row[rope_partner(d, half, rope_dim)];
            const int i = rope_index(d, half, rope_dim);
            c[e] = cs[i];
            s[e] = sn[i];
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

// Combine the 4 wave partials of one split (s_m, s_l, s_acc in LDS, after a
// workgroup barrier) and either finish the output (single split), store the
// split partial for decode_merge_kernel, or merge inline when this is the
// last split of its kv head.
struct SplitLds {
    float (*m)[kGroup];
    float (*l)[kGroup];
    float (*acc)[kGroup][kHeadDim];
    float (*w)[kMaxSplits];
    float *L;
    uint32_t *ticket;
};

__device__ __forceinline__ void split_epilogue(const DecodeArgs &a, int kvh, int split, int tid,
                                               const SplitLds &sl) {
    constexpr int D = kHeadDim, G = kGroup;
    auto &s_m = sl.m;
    auto &s_l = sl.l;
    auto &s_acc = sl.acc;
    auto &s_w = sl.w;
    float *s_L = sl.L;
    uint32_t &s_ticket = *sl.ticket;
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
        const int phys = a.pages_in_args ? a.pages[page] : a.tab[page];
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
        const int phys = a.pages_in_args ? a.pages[newpos / P] : a.tab[newpos / P];
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
    split_epilogue(a, kvh, split, tid, SplitLds{s_m, s_l, s_acc, s_w, s_L, &s_ticket});
}

// ---------------------------------------------------------------------------
// f16 / bf16 caches: the two dot products run on MFMA.
//   S  = K_sub (16 pos x 128) . Qcat^T      v_mfma_f32_16x16x32_{f16,bf16} x4
//   O += Pcat (16 rows x 16 pos) . V_sub     v_mfma_f32_16x16x16{f16,bf16_1k} x8
// Qcat columns 0..3 hold q of the 4 heads rounded to the operand type and
// columns 4..7 the rounding residual (q - hi) rounded again; Pcat rows 0..3 /
// 4..7 do the same for the softmax weights.  Summing the two halves gives
// q and P to about 2^-22 (f16) or 2^-18 (bf16) relative, i.e. the fp32 path's
// accuracy, with K and V consumed exactly as stored.
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

template <typename T, bool MULTI>
__global__ __launch_bounds__(256) void decode_attn_mfma_kernel(DecodeArgs a) {
    constexpr int D = kHeadDim, G = kGroup, P = kPage, SUB = 16;
    using M = DecMfma<T>;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, c = lane & 15;  // MFMA lane group / row-col index
    const int Hkv = a.kv_heads;
    const int kvh = blockIdx.x % Hkv;
    const int split = blockIdx.x / Hkv;
    const int npages = (a.L + P - 1) / P;
    const int page0 = split * a.ppw;
    const int page_end = MULTI ? min(page0 + a.ppw, npages) : page0 + 1;
    const int newpos = a.L - 1;
    const bool owner = page_end == npages;

    __shared__ float s_q[G][D];
    __shared__ __attribute__((aligned(16))) uint16_t s_knew[D];
    __shared__ uint16_t s_vnew[D];
    __shared__ float s_acc[4][G][D];
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_w[G][kMaxSplits];
    __shared__ float s_L[G];
    __shared__ uint32_t s_ticket;

    const size_t page_elems = (size_t)P * D;
    const uint16_t *kpool = (const uint16_t *)a.kpool;
    const uint16_t *vpool = (const uint16_t *)a.vpool;
    const int half = a.rope_half, rdim = a.rope_dim;

    RowIn qin, nin;
    qin.load(a.q + (size_t)(kvh * G + wave) * D, a.rope_cos, a.rope_sin, a.qnw, lane, half, rdim);
    if (owner && wave == 0)
        nin.load(a.knew + (size_t)kvh * D, a.rope_cos, a.rope_sin, a.knw, lane, half, rdim);
    if (owner && wave == 1)
        nin.load(a.vnew + (size_t)kvh * D, a.rope_cos, a.rope_sin, nullptr, lane, half, rdim);

    // K A-operand: lane (grp, c) = K row c, dims 32*ks + 8*grp + [0, 8)
    // V B-operand: lane (grp, c) = V^T row 16*db + c, positions 4*grp + [0, 4)
    uint4 ka[4], kn[4];
    uint2 vb[8], vn[8];
    auto load_sub = [&](int page, uint4 *kk, uint2 *vv) {
        const int base = page * P + SUB * wave;
        const int inmem = newpos - base;  // rows < inmem are resident
        const int phys = a.pages_in_args ? a.pages[page] : a.tab[page];
        const uint16_t *kp = kpool + ((size_t)phys * Hkv + kvh) * page_elems + (size_t)(SUB * wave) * D;
        const uint16_t *vp = vpool + ((size_t)phys * Hkv + kvh) * page_elems + (size_t)wave * D * SUB;
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
            kk[ks] = c < inmem ? *(const uint4 *)(kp + (size_t)c * D + 32 * ks + 8 * grp) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int db = 0; db < 8; db++)
            vv[db] = 4 * grp < inmem ? *(const uint2 *)(vp + (size_t)(16 * db + c) * SUB + 4 * grp) : make_uint2(0, 0);
    };
    load_sub(page0, ka, vb);
    if (MULTI && page0 + 1 < page_end) load_sub(page0 + 1, kn, vn);  // two pages in flight

    {
        float y[2];
        qin.finish(y, lane, half, rdim, a.qnw != nullptr, a.eps);
        s_q[wave][lane] = y[0] * a.qscale;
        s_q[wave][lane + 64] = y[1] * a.qscale;
    }
    if (owner && wave < 2) {
        const int t = newpos % P;
        const int phys = a.pages_in_args ? a.pages[newpos / P] : a.tab[newpos / P];
        if (wave == 0) {
            float y[2];
            nin.finish(y, lane, half, rdim, a.knw != nullptr, a.eps);
            uint16_t *kp = (uint16_t *)kpool + ((size_t)phys * Hkv + kvh) * page_elems + (size_t)t * D;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint16_t st = to_elem<T>(y[e]);
                kp[lane + 64 * e] = st;
                s_knew[lane + 64 * e] = st;
            }
        } else {
            uint16_t *vp = (uint16_t *)vpool + ((size_t)phys * Hkv + kvh) * page_elems;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
                const uint16_t st = to_elem<T>(nin.x[e]);
                vp[v_off(t, d)] = st;
                s_vnew[d] = st;
            }
        }
    }
    __syncthreads();

    // Qcat B-operand: lane (grp, c), dims 32*ks + 8*grp + [0, 8):
    // c < 4 -> hi(q_c), 4 <= c < 8 -> lo(q_{c-4}), else 0
    uint4 qb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (c < 8) {
            const float *qrow = s_q[c & 3] + 32 * ks + 8 * grp;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t p0 = split_pair<T>(qrow[2 * e]), p1 = split_pair<T>(qrow[2 * e + 1]);
                w[e] = c < 4 ? (p0 & 0xFFFFu) | (p1 << 16) : (p0 >> 16) | (p1 & 0xFFFF0000u);
            }
        }
        qb[ks] = make_uint4(w[0], w[1], w[2], w[3]);
    }

    f32x4 acc[8];
#pragma unroll
    for (int db = 0; db < 8; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kFloor2, l_run = 0.0f;  // lanes c < 4: head c

    for (int page = page0; page < page_end; page++) {
        const int base = page * P + SUB * wave;
        if (base < a.L) {
            const int rel = newpos - base;  // row of the new token in this sub-tile
            if (c == rel) {                 // new K row: the rounded value just appended
#pragma unroll
                for (int ks = 0; ks < 4; ks++) ka[ks] = *(const uint4 *)(s_knew + 32 * ks + 8 * grp);
            }
            // ---- scores: lane (grp, c<4) <- head c, positions 4*grp + i ----
            f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) sacc = M::qk(ka[ks], qb[ks], sacc);
            float sc[4], mt = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[i] = sacc[i] + dpp_from_plus4(sacc[i]);
                if (4 * grp + i <= rel) mt = fmaxf(mt, sc[i]);
            }
            mt = xrow32_max(xrow16_max(mt));
            const float mnew = fmaxf(m_run, mt);
            const float alpha = exp2f(m_run - mnew);
            float p[4], ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[i] = 4 * grp + i <= rel ? exp2f(fmaxf(sc[i] - mnew, kFloor2)) : 0.0f;
                ps += p[i];
            }
            ps = xrow32_sum(xrow16_sum(ps));
            l_run = l_run * alpha + ps;
            m_run = mnew;
            // ---- Pcat A-operand: lane (grp, r): r<4 hi(p_r), 4<=r<8 lo(p_{r-4}) ----
            uint32_t hp[2], lp[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t p0 = split_pair<T>(p[2 * e]), p1 = split_pair<T>(p[2 * e + 1]);
                hp[e] = (p0 & 0xFFFFu) | (p1 << 16);
                lp[e] = dpp_from_minus4((p0 >> 16) | (p1 & 0xFFFF0000u));
            }
            const uint2 pa = c < 4 ? make_uint2(hp[0], hp[1]) : c < 8 ? make_uint2(lp[0], lp[1]) : make_uint2(0u, 0u);
            // ---- V: zero positions past the new token, substitute the new row ----
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; i++) al[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), i));  // head i
#pragma unroll
            for (int db = 0; db < 8; db++) {
                uint2 v = vb[db];
                if (4 * grp + 3 >= rel) {
                    uint16_t e4[4] = {(uint16_t)(v.x & 0xFFFFu), (uint16_t)(v.x >> 16), (uint16_t)(v.y & 0xFFFFu), (uint16_t)(v.y >> 16)};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int r = 4 * grp + j;
                        if (r == rel) e4[j] = s_vnew[16 * db + c];
                        else if (r > rel) e4[j] = 0;
                    }
                    v = make_uint2(e4[0] | ((uint32_t)e4[1] << 16), e4[2] | ((uint32_t)e4[3] << 16));
                }
                f32x4 o = acc[db];
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] *= al[i];
                acc[db] = M::pv(pa, v, o);
            }
        }
        if (MULTI && page + 1 < page_end) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) ka[ks] = kn[ks];
#pragma unroll
            for (int db = 0; db < 8; db++) vb[db] = vn[db];
            if (page + 2 < page_end) load_sub(page + 2, kn, vn);
        }
    }

    // ---- wave partial: O[head i][16*db + c] = rows i (hi) + rows 4+i (lo) ----
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float o = xrow16_sum(acc[db][i]);
            if (grp == 0) s_acc[wave][i][16 * db + c] = o;
        }
    if (lane < G) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = l_run;
    }
    __syncthreads();
    split_epilogue(a, kvh, split, tid, SplitLds{s_m, s_l, s_acc, s_w, s_L, &s_ticket});
}

// Merge of the split partials (second launch when merge_inline is off).
// Block (head h, 32-dim slice); thread (split group sg of 8, dim).  Every
// thread issues all its (m, l, acc) loads at once, reduces its splits with a
// local maximum, and the 8 split groups are combined through LDS.
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    constexpr int D = kHeadDim, NG = 8, PER = kMaxSplits / NG;
    const int h = blockIdx.x >> 2, d = (blockIdx.x & 3) * 32 + (threadIdx.x & 31);
    const int sg = threadIdx.x >> 5;
    __shared__ float s_m[NG][32], s_l[NG][32], s_o[NG][32];
    const float *ml = a.part_ml + (size_t)h * kMaxSplits * 2;
    const float *pa = a.part_acc + (size_t)h * kMaxSplits * D + d;
    float m[PER], l[PER], x[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int s = sg + NG * k;
        const bool ok = s < a.nsplit;
        m[k] = ok ? ml[2 * s] : -INFINITY;
        l[k] = ok ? ml[2 * s + 1] : 0.0f;
        x[k] = ok ? pa[(size_t)s * D] : 0.0f;
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; k++) M = fmaxf(M, m[k]);
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const float w = exp2f(m[k] - M);
            L = fmaf(w, l[k], L);
            O = fmaf(w, x[k], O);
        }
    }
    s_m[sg][threadIdx.x & 31] = M;
    s_l[sg][threadIdx.x & 31] = L;
    s_o[sg][threadIdx.x & 31] = O;
    __syncthreads();
    if (sg == 0) {
        const int i = threadIdx.x & 31;
        float Mt = s_m[0][i];
#pragma unroll
        for (int g = 1; g < NG; g++) Mt = fmaxf(Mt, s_m[g][i]);
        float Lt = 0.0f, Ot = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            if (s_m[g][i] == -INFINITY) continue;
            const float w = exp2f(s_m[g][i] - Mt);
            Lt = fmaf(w, s_l[g][i], Lt);
            Ot = fmaf(w, s_o[g][i], Ot);
        }
        a.out[(size_t)h * D + d] = Lt > 0.0f ? Ot / Lt : 0.0f;
    }
}

hipError_t launch_decode(int kv_dtype, const DecodeArgs &a, hipStream_t s) {
    dim3 grid(a.nsplit * a.kv_heads), block(256);
    const bool multi = a.ppw > 1;
    switch (kv_dtype * 2 + multi) {
    case 0: hipLaunchKernelGGL((decode_attn_kernel<F32, false>), grid, block, 0, s, a); break;
    case 1: hipLaunchKernelGGL((decode_attn_kernel<F32, true>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((decode_attn_mfma_kernel<F16, false>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((decode_attn_mfma_kernel<F16, true>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((decode_attn_mfma_kernel<BF16, false>), grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL((decode_attn_mfma_kernel<BF16, true>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1 || a.merge_inline) return e;
    hipLaunchKernelGGL(decode_merge_kernel, dim3(a.kv_heads * kGroup * 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hymt
