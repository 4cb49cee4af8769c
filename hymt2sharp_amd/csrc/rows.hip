// rows.hip -- row-wise kernels between the prefill GEMMs (gfx950): RMSNorm of
// the residual rows into bf16 GEMM operands, SiLU(gate) * up into bf16, and
// plain fp32 -> bf16 rounding.  All are HBM-bound streaming kernels: every
// element is read once and written once, with 16-byte loads.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

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

// As rows_rmsnorm_kernel for rows of n <= 64 NJ float4s (n <= 4096): one
// wave per RPW rows, 4 waves per workgroup.  Every load (the rows' float4s
// and gamma's, gamma once for the RPW rows) is issued unconditionally before
// the first use -- past the row end a lane reloads the last float4 and counts
// nothing -- so the loads share one memory round trip; the row sum is a wave
// reduction, no barrier.
template <int NJ, int RPW>
__global__ __launch_bounds__(256) void rows_rmsnorm_wave_kernel(const float *__restrict__ x, int m, int n,
                                                                const float *__restrict__ w, float eps,
                                                                uint16_t *__restrict__ out) {
    const int lane = threadIdx.x & 63, n4 = n / 4;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
    float4 v[RPW][NJ], g[NJ];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const float4 *xr = (const float4 *)(x + (size_t)min(row0 + r, m - 1) * n);
#pragma unroll
        for (int j = 0; j < NJ; j++) v[r][j] = xr[min(lane + 64 * j, n4 - 1)];
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) g[j] = ((const float4 *)w)[min(lane + 64 * j, n4 - 1)];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; j++)
            if (lane + 64 * j < n4)
                ss += (v[r][j].x * v[r][j].x + v[r][j].y * v[r][j].y) + (v[r][j].z * v[r][j].z + v[r][j].w * v[r][j].w);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
        const float rr = 1.0f / sqrtf(ss / (float)n + eps);
        if (row0 + r >= m) continue;
        uint2 *orow = (uint2 *)(out + (size_t)(row0 + r) * n);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int i = lane + 64 * j;
            if (i < n4)
                orow[i] = pack4(v[r][j].x * rr * g[j].x, v[r][j].y * rr * g[j].y, v[r][j].z * rr * g[j].z,
                                v[r][j].w * rr * g[j].w);
        }
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

// As rows_swiglu_bf16_kernel with 16-byte accesses (8 values) when n is a
// multiple of 8 and the buffers are 16-byte aligned, with 32-bit index
// arithmetic (the launcher checks m n / 8 <= 2^30, so e plus the grid stride
// stays below 2^31) and swiglu8 (silu_fast): the exact quotient's exp and
// division were most of its time.  The gate/up GEMM's fused epilogue
// (gemm_mfma.hip) computes the same swiglu8 of the same bf16 values.
__global__ __launch_bounds__(256) void rows_swiglu_bf16_x8_kernel(const uint16_t *__restrict__ gu, int m, int n,
                                                                  uint16_t *__restrict__ out) {
    const int n8 = n / 8, total = m * n8;
    for (int e = blockIdx.x * 256 + threadIdx.x; e < total; e += gridDim.x * 256) {
        const int r = e / n8, i = e - r * n8;
        const uint4 gb = ((const uint4 *)(gu + (size_t)r * 2 * n))[i];
        const uint4 ub = ((const uint4 *)(gu + (size_t)r * 2 * n + n))[i];
        ((uint4 *)(out + (size_t)r * n))[i] = swiglu8(gb, ub);
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
    const int nj = (n / 4 + 63) / 64;  // float4s per lane with a wave per row
    auto wave_rows = [&](auto nj_tag, auto rpw_tag) {
        constexpr int NJ = decltype(nj_tag)::value, RPW = decltype(rpw_tag)::value;
        const unsigned blocks = (unsigned)(((size_t)m + 4 * RPW - 1) / (4 * RPW));
        launch(span, rows_rmsnorm_wave_kernel<NJ, RPW>, dim3(blocks), dim3(256), 0, s, x, m, n, w, eps, out);
    };
    using I = std::integral_constant<int, 1>;
    using II = std::integral_constant<int, 2>;
    if (nj <= 1) wave_rows(std::integral_constant<int, 1>{}, II{});
    else if (nj <= 2) wave_rows(std::integral_constant<int, 2>{}, II{});
    else if (nj <= 4) wave_rows(std::integral_constant<int, 4>{}, II{});
    else if (nj <= 8) wave_rows(std::integral_constant<int, 8>{}, II{});
    else if (nj <= 16) wave_rows(std::integral_constant<int, 16>{}, I{});
    else launch(span, rows_rmsnorm_kernel, dim3(m), dim3(256), 0, s, x, n, w, eps, out);
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
    if (n % 8 == 0 && ((uintptr_t)gu & 15u) == 0 && ((uintptr_t)out & 15u) == 0 && (size_t)m * (n / 8) <= (1u << 30))
        launch(span, rows_swiglu_bf16_x8_kernel, dim3(grid_for((size_t)m * n / 8)), dim3(256), 0, s, gu, m, n, out);
    else
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
