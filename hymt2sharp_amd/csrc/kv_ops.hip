// kv_ops.hip -- page-table mirroring and bulk K/V row transfers for the
// paged cache (layout in attn_kernels.hpp).
#include <algorithm>

#include "attn_kernels.hpp"
#include "device_common.hpp"
#include "ktimer.hpp"

namespace hymt {

// Up to 64 table entries per launch, passed by value so the host copy can
// change as soon as the launch returns.
struct TabUpdate {
    int n;
    int idx[64];
    int val[64];
};

__global__ void tab_update_kernel(int32_t *tab, TabUpdate u) {
    int i = threadIdx.x;
    if (i < u.n) tab[u.idx[i]] = u.val[i];
}

hipError_t launch_tab_update(int32_t *tab, const int *idx, const int *val, int n, hipStream_t s) {
    KernelSpan span("tab_update", s);
    for (int off = 0; off < n; off += 64) {
        TabUpdate u;
        u.n = n - off < 64 ? n - off : 64;
        for (int i = 0; i < u.n; i++) {
            u.idx[i] = idx[off + i];
            u.val[i] = val[off + i];
        }
        hipLaunchKernelGGL(tab_update_kernel, dim3(1), dim3(64), 0, s, tab, u);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Copy-on-write of one page for the block store (MetalBackend.cs
// ExecCopies, :320-332, its kv_copy_block kernel): page src -> page dst in
// every layer's K and V pool.  A page of all kv heads is one contiguous
// block of page_bytes, copied as 16-byte vectors; grid.y = (layer, K/V).
__global__ __launch_bounds__(256) void kv_copy_page_kernel(uint4 *kpool, uint4 *vpool, size_t layer_vec,
                                                           size_t page_vec, int src, int dst) {
    uint4 *pool = (blockIdx.y & 1) ? vpool : kpool;
    const size_t base = (size_t)(blockIdx.y >> 1) * layer_vec;
    const uint4 *from = pool + base + (size_t)src * page_vec;
    uint4 *to = pool + base + (size_t)dst * page_vec;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < page_vec; i += (size_t)gridDim.x * blockDim.x)
        to[i] = from[i];
}

hipError_t launch_kv_copy_page(void *kpool, void *vpool, size_t layer_bytes, size_t page_bytes, int src,
                               int dst, int layers, hipStream_t s) {
    if (src == dst || layers <= 0) return hipSuccess;
    const size_t page_vec = page_bytes / 16;
    const int bx = (int)std::min<size_t>((page_vec + 255) / 256, 64);
    KernelSpan span("kv_copy_page", s);
    hipLaunchKernelGGL(kv_copy_page_kernel, dim3(bx, 2 * layers), dim3(256), 0, s, (uint4 *)kpool,
                       (uint4 *)vpool, layer_bytes / 16, page_vec, src, dst);
    return hipGetLastError();
}

// IComputeBackend.UploadKv (IComputeBackend.cs:31-38): rows [pos, pos+len)
// of flat bf16 [row][Hkv*D] caches (kb/vb point at row pos) -> paged cache
// in its dtype.  One thread per (row, kvh, d).
template <typename T>
__global__ void kv_upload_kernel(const uint16_t *kb, const uint16_t *vb, const int32_t *tab,
                                 typename T::storage *kpool, typename T::storage *vpool, int pos,
                                 int len, int Hkv) {
    constexpr int D = kHeadDim, P = kPage;
    const long n = (long)len * Hkv * D;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
        const int d = (int)(i % D);
        const int kvh = (int)((i / D) % Hkv);
        const int j = pos + (int)(i / ((long)D * Hkv));
        const int phys = tab[j / P], t = j % P;
        const size_t pg = ((size_t)phys * Hkv + kvh) * (size_t)(P * D);
        const size_t src = (size_t)(j - pos) * Hkv * D + (size_t)kvh * D + d;
        constexpr int B = sizeof(typename T::storage);
        kpool[pg + k_off<B>(t, d)] = to_elem<T>(bf16_to_f32(kb[src]));
        vpool[pg + v_off<B>(t, d)] = to_elem<T>(bf16_to_f32(vb[src]));
    }
}

hipError_t launch_kv_upload(int kv_dtype, const uint16_t *k_bf16, const uint16_t *v_bf16,
                            const int32_t *tab, void *kpool, void *vpool, int pos, int len,
                            int kv_heads, hipStream_t s) {
    long n = (long)len * kv_heads * kHeadDim;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) return hipSuccess;
    KernelSpan span("kv_upload", s);
    switch (kv_dtype) {
    case 0: hipLaunchKernelGGL(kv_upload_kernel<F32>, dim3(blocks), dim3(256), 0, s, k_bf16, v_bf16, tab, (float *)kpool, (float *)vpool, pos, len, kv_heads); break;
    case 1: hipLaunchKernelGGL(kv_upload_kernel<F16>, dim3(blocks), dim3(256), 0, s, k_bf16, v_bf16, tab, (uint16_t *)kpool, (uint16_t *)vpool, pos, len, kv_heads); break;
    case 2: hipLaunchKernelGGL(kv_upload_kernel<BF16>, dim3(blocks), dim3(256), 0, s, k_bf16, v_bf16, tab, (uint16_t *)kpool, (uint16_t *)vpool, pos, len, kv_heads); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename T>
__global__ void kv_read_kernel(const int32_t *tab, const typename T::storage *kpool,
                               const typename T::storage *vpool, float *ko, float *vo, int pos,
                               int len, int Hkv) {
    constexpr int D = kHeadDim, P = kPage;
    const long n = (long)len * Hkv * D;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
        const int d = (int)(i % D);
        const int kvh = (int)((i / D) % Hkv);
        const int r = (int)(i / ((long)D * Hkv));
        const int j = pos + r;
        const int phys = tab[j / P], t = j % P;
        const size_t pg = ((size_t)phys * Hkv + kvh) * (size_t)(P * D);
        constexpr int B = sizeof(typename T::storage);
        ko[i] = from_elem<T>(kpool[pg + k_off<B>(t, d)]);
        vo[i] = from_elem<T>(vpool[pg + v_off<B>(t, d)]);
    }
}

hipError_t launch_kv_read(int kv_dtype, const int32_t *tab, const void *kpool, const void *vpool,
                          float *k_out, float *v_out, int pos, int len, int kv_heads,
                          hipStream_t s) {
    long n = (long)len * kv_heads * kHeadDim;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) return hipSuccess;
    KernelSpan span("kv_read", s);
    switch (kv_dtype) {
    case 0: hipLaunchKernelGGL(kv_read_kernel<F32>, dim3(blocks), dim3(256), 0, s, tab, (const float *)kpool, (const float *)vpool, k_out, v_out, pos, len, kv_heads); break;
    case 1: hipLaunchKernelGGL(kv_read_kernel<F16>, dim3(blocks), dim3(256), 0, s, tab, (const uint16_t *)kpool, (const uint16_t *)vpool, k_out, v_out, pos, len, kv_heads); break;
    case 2: hipLaunchKernelGGL(kv_read_kernel<BF16>, dim3(blocks), dim3(256), 0, s, tab, (const uint16_t *)kpool, (const uint16_t *)vpool, k_out, v_out, pos, len, kv_heads); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace hymt
