// rows.hip -- row-wise kernels between the prefill GEMMs (gfx950): RMSNorm of
// the residual rows into bf16 GEMM operands, SiLU(gate) * up into bf16, and
// plain fp32 -> bf16 rounding.  All are HBM-bound streaming kernels: every
// element is read once and written once, with 16-byte loads.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"
#include "ktimer.hpp"
#include "weights.hpp"

namespace hymt {
namespace {

__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
    return make_uint2((uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16),
                      (uint32_t)f32_to_bf16(c) | ((uint32_t)f32_to_bf16(d) << 16));
}

// out[r] = x[r] / sqrt(mean(x[r]^2) + eps) * w (Ops.RmsNorm, Ops.cs:12-90):
// one workgroup per row, the row held in registers (n <= 8192).
__global__ __launch_bounds__(256) void rows_rmsnorm_kernel(const float *__restrict__ x, int n,
                                                           const float *__restrict__ w, float eps,
                                                           uint16_t *__restrict__ out) {
    constexpr int kMax = 8;  // float4s per thread: n <= 8192
    const int tid = threadIdx.x, n4 = n / 4;
    const float4 *xr = (const float4 *)(x + (size_t)blockIdx.x * n);
    float4 v[kMax], g[kMax];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kMax; j++) {
        const int i = tid + 256 * j;
        if (i < n4) {
            v[j] = xr[i];
            g[j] = ((const float4 *)w)[i];
        }
    }
#pragma unroll
    for (int j = 0; j < kMax; j++)
        if (tid + 256 * j < n4) ss += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    __shared__ float red[4];
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float rr = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)n + eps);
    uint2 *orow = (uint2 *)(out + (size_t)blockIdx.x * n);
#pragma unroll
    for (int j = 0; j < kMax; j++) {
        const int i = tid + 256 * j;
        if (i < n4)
            orow[i] = pack4(v[j].x * rr * g[j].x, v[j].y * rr * g[j].y, v[j].z * rr * g[j].z, v[j].w * rr * g[j].w);
    }
}

// out[r][i] = g / (1 + exp(-g)) * u with g = gu[r][i], u = gu[r][n + i]
// (Ops.SiLUMulRange, Ops.cs:1016-1052)
__global__ __launch_bounds__(256) void rows_swiglu_kernel(const float *__restrict__ gu, int m, int n,
                                                          uint16_t *__restrict__ out) {
    const int n4 = n / 4;
    const size_t total = (size_t)m * n4;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (size_t)gridDim.x * 256) {
        const size_t r = e / n4, i = e % n4;
        const float4 g = ((const float4 *)(gu + r * 2 * n))[i], u = ((const float4 *)(gu + r * 2 * n + n))[i];
        ((uint2 *)(out + r * n))[i] = pack4(g.x / (1.f + expf(-g.x)) * u.x, g.y / (1.f + expf(-g.y)) * u.y,
                                            g.z / (1.f + expf(-g.z)) * u.z, g.w / (1.f + expf(-g.w)) * u.w);
    }
}

// As rows_swiglu_kernel over a bf16 gate/up GEMM output (half the bytes).
__global__ __launch_bounds__(256) void rows_swiglu_bf16_kernel(const uint16_t *__restrict__ gu, int m, int n,
                                                               uint16_t *__restrict__ out) {
    const int n4 = n / 4;
    const size_t total = (size_t)m * n4;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (size_t)gridDim.x * 256) {
        const size_t r = e / n4, i = e % n4;
        const uint2 gb = ((const uint2 *)(gu + r * 2 * n))[i], ub = ((const uint2 *)(gu + r * 2 * n + n))[i];
        const float g[4] = {bf16_to_f32(gb.x & 0xFFFF), bf16_to_f32(gb.x >> 16), bf16_to_f32(gb.y & 0xFFFF),
                            bf16_to_f32(gb.y >> 16)};
        const float u[4] = {bf16_to_f32(ub.x & 0xFFFF), bf16_to_f32(ub.x >> 16), bf16_to_f32(ub.y & 0xFFFF),
                            bf16_to_f32(ub.y >> 16)};
        ((uint2 *)(out + r * n))[i] = pack4(g[0] / (1.f + expf(-g[0])) * u[0], g[1] / (1.f + expf(-g[1])) * u[1],
                                            g[2] / (1.f + expf(-g[2])) * u[2], g[3] / (1.f + expf(-g[3])) * u[3]);
    }
}

__global__ __launch_bounds__(256) void to_bf16_kernel(const float *__restrict__ x, size_t n4,
                                                      uint16_t *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const float4 v = ((const float4 *)x)[i];
        ((uint2 *)out)[i] = pack4(v.x, v.y, v.z, v.w);
    }
}

unsigned grid_for(size_t items) {
    const size_t g = (items + 255) / 256;
    return (unsigned)(g < 4096 ? (g ? g : 1) : 4096);
}

}  // namespace

hipError_t launch_rows_rmsnorm(const float *x, int m, int n, const float *w, float eps, uint16_t *out,
                               hipStream_t s) {
    if (n % 4 != 0 || n > 8192 || m < 0) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    KernelSpan span("rows_rmsnorm", s, true);
    launch(span, rows_rmsnorm_kernel, dim3(m), dim3(256), 0, s, x, n, w, eps, out);
    return hipGetLastError();
}

hipError_t launch_rows_swiglu(const float *gu, int m, int n, uint16_t *out, hipStream_t s) {
    if (n % 4 != 0 || m < 0) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    KernelSpan span("rows_swiglu", s, true);
    launch(span, rows_swiglu_kernel, dim3(grid_for((size_t)m * n / 4)), dim3(256), 0, s, gu, m, n, out);
    return hipGetLastError();
}

hipError_t launch_rows_swiglu_bf16(const uint16_t *gu, int m, int n, uint16_t *out, hipStream_t s) {
    if (n % 4 != 0 || m < 0) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    KernelSpan span("rows_swiglu_bf16", s, true);
    launch(span, rows_swiglu_bf16_kernel, dim3(grid_for((size_t)m * n / 4)), dim3(256), 0, s, gu, m, n, out);
    return hipGetLastError();
}

hipError_t launch_to_bf16(const float *x, size_t count, uint16_t *out, hipStream_t s) {
    if (count % 4 != 0) return hipErrorInvalidValue;
    if (count == 0) return hipSuccess;
    KernelSpan span("to_bf16", s, true);
    launch(span, to_bf16_kernel, dim3(grid_for(count / 4)), dim3(256), 0, s, x, count / 4, out);
    return hipGetLastError();
}

}  // namespace hymt
