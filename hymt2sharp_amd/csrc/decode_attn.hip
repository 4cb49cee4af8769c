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
// MslDecodeKernels.cs:172-300, but over KV heads so each K/V byte is read
// from HBM exactly once for all 4 q heads of its GQA group):
//   workgroup (split, kvh), 256 threads, `ppw` 64-token pages per split.
//   Each split produces (m, l, acc[128]) per q head; the last workgroup of a
//   kv head to finish (atomic ticket) merges the splits and writes out.
// Loads are 16-byte vectors: a K page row (128 elems) is 16 lanes, a V^T page
// row (64 positions) 8 lanes, so one wave-wide load covers 1 KiB contiguous.
#include "attn_kernels.hpp"
#include "device_common.hpp"

namespace hymt {

template <typename T>
__global__ __launch_bounds__(256) void decode_attn_kernel(DecodeArgs a) {
    constexpr int D = kHeadDim, G = kGroup, P = kPage;
    using S = typename T::storage;
    constexpr int VN = Vec16<T>::N;   // elements per 16-byte vector
    constexpr int KCPR = D / VN;      // K vectors per row
    constexpr int KROWS = 256 / KCPR; // rows per pass
    constexpr int KPASS = P / KROWS;
    constexpr int VCPR = P / VN;      // V^T vectors per d row
    constexpr int VROWS = 256 / VCPR;
    constexpr int VPASS = D / VROWS;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Hkv = a.kv_heads;
    const int kvh = blockIdx.x % Hkv;
    const int split = blockIdx.x / Hkv;
    const int npages = (a.L + P - 1) / P;
    const int page0 = split * a.ppw;
    const int page_end = min(page0 + a.ppw, npages);
    const int newpos = a.L - 1;
    const bool owner = page_end == npages;

    __shared__ float s_q[G][D];
    __shared__ float s_knew[D], s_vnew[D];
    __shared__ float s_p[G][P];
    __shared__ float s_alpha[G], s_l[G];
    __shared__ float s_w[G][kMaxSplits];
    __shared__ uint32_t s_ticket;

    const S *kpool = (const S *)a.kpool;
    const S *vpool = (const S *)a.vpool;
    const size_t page_elems = (size_t)P * D;  // per (page, kvh)

    const int kc = tid % KCPR, kr0 = tid / KCPR;
    const int vc = tid % VCPR, vd0 = tid / VCPR;

    // ---- issue the first page's loads before the prologue math ----------
    uint4 kb[KPASS], vb[VPASS];
    auto load_page = [&](int page, uint4 *kk, uint4 *vv) {
        const int base = page * P;
        const int valid = min(P, newpos - base);  // rows < newpos come from memory
        const int phys = a.tab[page];
        const S *kp = kpool + ((size_t)phys * Hkv + kvh) * page_elems;
        const S *vp = vpool + ((size_t)phys * Hkv + kvh) * page_elems;
#pragma unroll
        for (int j = 0; j < KPASS; j++) {
            const int r = kr0 + KROWS * j;
            kk[j] = r < valid ? *(const uint4 *)(kp + (size_t)r * D + kc * VN) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < VPASS; j++) {
            const int d = vd0 + VROWS * j;
            vv[j] = vc * VN < valid ? *(const uint4 *)(vp + (size_t)d * P + vc * VN) : make_uint4(0, 0, 0, 0);
        }
    };
    load_page(page0, kb, vb);

    // ---- prologue: RoPE + RMSNorm of the group's q heads ----------------
    {
        const int h = kvh * G + wave;
        const float *qh = a.q + (size_t)h * D;
        float y[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int d = lane + 64 * e;
            float x = qh[d];
            if (d < a.rope_half) {
                y[e] = x * a.rope_cos[d] - qh[d + a.rope_half] * a.rope_sin[d];
            } else if (d < a.rope_dim) {
                const int i = d - a.rope_half;
                y[e] = qh[i] * a.rope_sin[i] + x * a.rope_cos[i];
            } else {
                y[e] = x;
            }
        }
        if (a.qnw) {
            float ss = group_sum<64>(y[0] * y[0] + y[1] * y[1]);
            float r = 1.0f / sqrtf(ss / (float)D + a.eps);
            y[0] = y[0] * r * a.qnw[lane];
            y[1] = y[1] * r * a.qnw[lane + 64];
        }
        s_q[wave][lane] = y[0] * a.qscale;
        s_q[wave][lane + 64] = y[1] * a.qscale;
    }
    if (owner && wave < 2) {
        // wave 0: new K row (RoPE + norm, rounded); wave 1: new V row (rounded)
        const int page = newpos / P, row = newpos % P;
        const int phys = a.tab[page];
        if (wave == 0) {
            const float *kh = a.knew + (size_t)kvh * D;
            float y[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
                float x = kh[d];
                if (d < a.rope_half) {
                    y[e] = x * a.rope_cos[d] - kh[d + a.rope_half] * a.rope_sin[d];
                } else if (d < a.rope_dim) {
                    const int i = d - a.rope_half;
                    y[e] = kh[i] * a.rope_sin[i] + x * a.rope_cos[i];
                } else {
                    y[e] = x;
                }
            }
            if (a.knw) {
                float ss = group_sum<64>(y[0] * y[0] + y[1] * y[1]);
                float r = 1.0f / sqrtf(ss / (float)D + a.eps);
                y[0] = y[0] * r * a.knw[lane];
                y[1] = y[1] * r * a.knw[lane + 64];
            }
            S *kp = (S *)kpool + ((size_t)phys * Hkv + kvh) * page_elems + (size_t)row * D;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
                S st = to_elem<T>(y[e]);
                kp[d] = st;
                s_knew[d] = from_elem<T>(st);
            }
        } else {
            const float *vh = a.vnew + (size_t)kvh * D;
            S *vp = (S *)vpool + ((size_t)phys * Hkv + kvh) * page_elems + row;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = lane + 64 * e;
                S st = to_elem<T>(vh[d]);
                vp[(size_t)d * P] = st;
                s_vnew[d] = from_elem<T>(st);
            }
        }
    }
    __syncthreads();

    // q chunk this thread multiplies K vectors with (same for every row)
    float qreg[G][VN];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < VN; e++) qreg[g][e] = s_q[g][kc * VN + e];

    float acc[VPASS][G];
#pragma unroll
    for (int j = 0; j < VPASS; j++)
#pragma unroll
        for (int g = 0; g < G; g++) acc[j][g] = 0.0f;
    float m_run = kFloor2, l_run = 0.0f;  // wave `wave` tracks head `wave`

    for (int page = page0; page < page_end; page++) {
        const int base = page * P;
        const int nvalid = min(P, a.L - base);
        uint4 kn[KPASS], vn[VPASS];
        const bool more = page + 1 < page_end;
        if (more) load_page(page + 1, kn, vn);

        // ---- scores: rows kr0 + KROWS*j --------------------------------
#pragma unroll
        for (int j = 0; j < KPASS; j++) {
            const int r = kr0 + KROWS * j;
            float kv[VN];
            Vec16<T>::unpack(kb[j], kv);
            if (base + r == newpos) {
#pragma unroll
                for (int e = 0; e < VN; e++) kv[e] = s_knew[kc * VN + e];
            }
            float dot[G];
#pragma unroll
            for (int g = 0; g < G; g++) {
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < VN; e++) s = fmaf(qreg[g][e], kv[e], s);
                dot[g] = group_sum<KCPR>(s);
            }
            if (kc == 0) {
#pragma unroll
                for (int g = 0; g < G; g++) s_p[g][r] = r < nvalid ? dot[g] : -INFINITY;
            }
        }
        __syncthreads();

        // ---- online softmax per head (wave g <-> head g) ----------------
        {
            const float s = s_p[wave][lane];
            const float mt = group_max<64>(s);
            const float m_new = fmaxf(m_run, mt);
            const float p = lane < nvalid ? exp2f(fmaxf(s - m_new, kFloor2)) : 0.0f;
            const float alpha = exp2f(m_run - m_new);
            l_run = l_run * alpha + group_sum<64>(p);
            m_run = m_new;
            s_p[wave][lane] = p;
            if (lane == 0) s_alpha[wave] = alpha;
        }
        __syncthreads();

        // ---- P * V over this page --------------------------------------
        {
            float preg[G][VN];
            float alpha[G];
#pragma unroll
            for (int g = 0; g < G; g++) {
                alpha[g] = s_alpha[g];
#pragma unroll
                for (int e = 0; e < VN; e++) preg[g][e] = s_p[g][vc * VN + e];
            }
#pragma unroll
            for (int j = 0; j < VPASS; j++) {
                const int d = vd0 + VROWS * j;
                float vv[VN];
                Vec16<T>::unpack(vb[j], vv);
#pragma unroll
                for (int e = 0; e < VN; e++) {
                    const int t = vc * VN + e;
                    if (base + t == newpos) vv[e] = s_vnew[d];
                    else if (t >= nvalid) vv[e] = 0.0f;
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    float s = acc[j][g] * alpha[g];
#pragma unroll
                    for (int e = 0; e < VN; e++) s = fmaf(preg[g][e], vv[e], s);
                    acc[j][g] = s;
                }
            }
        }
        if (more) {
#pragma unroll
            for (int j = 0; j < KPASS; j++) kb[j] = kn[j];
#pragma unroll
            for (int j = 0; j < VPASS; j++) vb[j] = vn[j];
            __syncthreads();  // s_p / s_alpha reuse by the next page
        }
    }

    // reduce the position chunks of each d row
#pragma unroll
    for (int j = 0; j < VPASS; j++)
#pragma unroll
        for (int g = 0; g < G; g++) acc[j][g] = group_sum<VCPR>(acc[j][g]);

    const int HqBase = kvh * G;
    if (a.nsplit == 1) {
        if (lane == 0) s_l[wave] = l_run;
        __syncthreads();
        if (vc == 0) {
#pragma unroll
            for (int j = 0; j < VPASS; j++) {
                const int d = vd0 + VROWS * j;
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float l = s_l[g];
                    a.out[(size_t)(HqBase + g) * D + d] = l > 0.0f ? acc[j][g] / l : 0.0f;
                }
            }
        }
        return;
    }

    // ---- write this split's partial, then the last split merges ----------
    if (vc == 0) {
#pragma unroll
        for (int j = 0; j < VPASS; j++) {
            const int d = vd0 + VROWS * j;
#pragma unroll
            for (int g = 0; g < G; g++)
                a.part_acc[((size_t)(HqBase + g) * kMaxSplits + split) * D + d] = acc[j][g];
        }
    }
    if (lane == 0) {
        float *ml = a.part_ml + ((size_t)(HqBase + wave) * kMaxSplits + split) * 2;
        ml[0] = m_run;
        ml[1] = l_run;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) s_ticket = atomicAdd(&a.counters[kvh], 1u);
    __syncthreads();
    if (s_ticket != (uint32_t)(a.nsplit - 1)) return;
    __threadfence();

    {
        // wave g merges head g's statistics
        const int h = HqBase + wave;
        const float *ml = a.part_ml + (size_t)h * kMaxSplits * 2;
        float mloc = -INFINITY;
        for (int s = lane; s < a.nsplit; s += 64) mloc = fmaxf(mloc, ml[2 * s]);
        const float M = group_max<64>(mloc);
        float lsum = 0.0f;
        for (int s = lane; s < a.nsplit; s += 64) {
            const float w = exp2f(ml[2 * s] - M);
            s_w[wave][s] = w;
            lsum += w * ml[2 * s + 1];
        }
        lsum = group_sum<64>(lsum);
        if (lane == 0) s_l[wave] = lsum;
    }
    __syncthreads();
    {
        const int g = wave, h = HqBase + g;
        const int d = lane * 2;
        const float *pa = a.part_acc + (size_t)h * kMaxSplits * D + d;
        float o0 = 0.0f, o1 = 0.0f;
        int s = 0;
        for (; s + 4 <= a.nsplit; s += 4) {
            float2 x0 = *(const float2 *)(pa + (size_t)(s + 0) * D);
            float2 x1 = *(const float2 *)(pa + (size_t)(s + 1) * D);
            float2 x2 = *(const float2 *)(pa + (size_t)(s + 2) * D);
            float2 x3 = *(const float2 *)(pa + (size_t)(s + 3) * D);
            o0 = fmaf(s_w[g][s + 0], x0.x, o0); o1 = fmaf(s_w[g][s + 0], x0.y, o1);
            o0 = fmaf(s_w[g][s + 1], x1.x, o0); o1 = fmaf(s_w[g][s + 1], x1.y, o1);
            o0 = fmaf(s_w[g][s + 2], x2.x, o0); o1 = fmaf(s_w[g][s + 2], x2.y, o1);
            o0 = fmaf(s_w[g][s + 3], x3.x, o0); o1 = fmaf(s_w[g][s + 3], x3.y, o1);
        }
        for (; s < a.nsplit; s++) {
            float2 x = *(const float2 *)(pa + (size_t)s * D);
            o0 = fmaf(s_w[g][s], x.x, o0);
            o1 = fmaf(s_w[g][s], x.y, o1);
        }
        const float l = s_l[g];
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        *(float2 *)(a.out + (size_t)h * D + d) = make_float2(o0 * inv, o1 * inv);
    }
    if (tid == 0) a.counters[kvh] = 0u;
}

hipError_t launch_decode(int kv_dtype, const DecodeArgs &a, hipStream_t s) {
    dim3 grid(a.nsplit * a.kv_heads), block(256);
    switch (kv_dtype) {
    case 0: hipLaunchKernelGGL(decode_attn_kernel<F32>, grid, block, 0, s, a); break;
    case 1: hipLaunchKernelGGL(decode_attn_kernel<F16>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(decode_attn_kernel<BF16>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace hymt
