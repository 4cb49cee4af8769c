// device_common.hpp -- element types, conversions and wave reductions shared
// by the gfx950 kernels of the attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hymt {

// Cache element tags.  Storage of F16 and BF16 is uint16_t bit patterns.
struct F32 {
    using storage = float;
    static constexpr int kBytes = 4;
};
struct F16 {
    using storage = uint16_t;
    static constexpr int kBytes = 2;
};
struct BF16 {
    using storage = uint16_t;
    static constexpr int kBytes = 2;
};

// fp32 -> bf16 with the reference's integer round-to-nearest-even
// (Ops.cs:664-665: no NaN special case).
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    uint32_t b = __float_as_uint(x);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> fp16 round-to-nearest-even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
    _Float16 h = (_Float16)x;
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <typename T> __device__ __forceinline__ typename T::storage to_elem(float x);
template <> __device__ __forceinline__ float to_elem<F32>(float x) { return x; }
template <> __device__ __forceinline__ uint16_t to_elem<F16>(float x) { return f32_to_f16(x); }
template <> __device__ __forceinline__ uint16_t to_elem<BF16>(float x) { return f32_to_bf16(x); }

template <typename T> __device__ __forceinline__ float from_elem(typename T::storage x);
template <> __device__ __forceinline__ float from_elem<F32>(float x) { return x; }
template <> __device__ __forceinline__ float from_elem<F16>(uint16_t x) { return f16_to_f32(x); }
template <> __device__ __forceinline__ float from_elem<BF16>(uint16_t x) { return bf16_to_f32(x); }

// Widen the elements packed in one 16-byte vector.
// F16/BF16: 8 elements; F32: 4 elements.
template <typename T> struct Vec16;
template <> struct Vec16<F32> {
    static constexpr int N = 4;
    __device__ static __forceinline__ void unpack(const uint4 &v, float *o) {
        o[0] = __uint_as_float(v.x);
        o[1] = __uint_as_float(v.y);
        o[2] = __uint_as_float(v.z);
        o[3] = __uint_as_float(v.w);
    }
};
template <> struct Vec16<BF16> {
    static constexpr int N = 8;
    __device__ static __forceinline__ void unpack(const uint4 &v, float *o) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = __uint_as_float(w[i] << 16);
            o[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
};
template <> struct Vec16<F16> {
    static constexpr int N = 8;
    __device__ static __forceinline__ void unpack(const uint4 &v, float *o) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xFFFFu));
            o[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
        }
    }
};

// Butterfly reductions over `width` consecutive lanes of a wave64.
template <int WIDTH> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int WIDTH> __device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over each row of 16 lanes with DPP (quad_perm xor 1, xor 2, then
// half-row and row mirrors); every lane of the row receives the sum.
__device__ __forceinline__ float dpp_sum16(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    return v;
}
// Sum over groups of 2 / 4 consecutive lanes (quad_perm).
__device__ __forceinline__ float dpp_sum2(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_sum4(float v) {
    v = dpp_sum2(v);
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}
// Sum over WIDTH consecutive lanes (WIDTH in 2, 4, 16, 32, 64): DPP inside a
// 16-lane row, a lane shuffle across rows.
template <int WIDTH> __device__ __forceinline__ float lane_sum(float v) {
    if constexpr (WIDTH == 2) return dpp_sum2(v);
    if constexpr (WIDTH == 4) return dpp_sum4(v);
    v = dpp_sum16(v);
#pragma unroll
    for (int o = 16; o < WIDTH; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// log2(e) and the softmax floor of Ops.SoftmaxRow (exp(max(x - max, -80)),
// Ops.cs:231,245,256) in base-2 units.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kFloor2 = -80.0f * 1.4426950408889634f;

}  // namespace hymt
