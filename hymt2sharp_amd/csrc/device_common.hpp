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

// silu(g) = g / (1 + e^-g) from the hardware's base-2 exponential and
// reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each): a few fp32 ulps from
// the correctly rounded quotient, far inside the bf16 rounding of the result.
// Large |g| behaves as the exact form: e^-g overflows to inf for g < -88 and
// gives -0, and underflows to 0 for large g and gives g.
__device__ __forceinline__ float silu_fast(float g) {
    return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
}

// bf16 silu(g) u of 8 bf16 gate values g and 8 up values u, 16 bytes each
// (Ops.SiLUMulRange, Ops.cs:1016-1052, over bf16 inputs)
__device__ __forceinline__ uint4 swiglu8(uint4 gb, uint4 ub) {
    const uint32_t gw[4] = {gb.x, gb.y, gb.z, gb.w};
    const uint32_t uw[4] = {ub.x, ub.y, ub.z, ub.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float g0 = bf16_to_f32(gw[k] & 0xFFFF), g1 = bf16_to_f32(gw[k] >> 16);
        const float u0 = bf16_to_f32(uw[k] & 0xFFFF), u1 = bf16_to_f32(uw[k] >> 16);
        o[k] = (uint32_t)f32_to_bf16(silu_fast(g0) * u0) | ((uint32_t)f32_to_bf16(silu_fast(g1) * u1) << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

template <typename T> __device__ __forceinline__ typename T::storage to_elem(float x);
template <> __device__ __forceinline__ float to_elem<F32>(float x) { return x; }
template <> __device__ __forceinline__ uint16_t to_elem<F16>(float x) { return f32_to_f16(x); }
template <> __device__ __forceinline__ uint16_t to_elem<BF16>(float x) { return f32_to_bf16(x); }

template <typename T> __device__ __forceinline__ float from_elem(typename T::storage x);
template <> __device__ __forceinline__ float from_elem<F32>(float x) { return x; }
template <> __device__ __forceinline__ float from_elem<F16>(uint16_t x) { return f16_to_f32(x); }
template <> __device__ __forceinline__ float from_elem<BF16>(uint16_t x) { return bf16_to_f32(x); }

// Sum over each row of 16 lanes with DPP (quad_perm xor 1, xor 2, then
// half-row and row mirrors); every lane of the row receives the sum.
__device__ __forceinline__ float dpp_sum16(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    return v;
}
// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane i writes LDS bytes lds_base + 16 i.
// Issued as inline assembly so that the compiler does not treat it as an LDS
// store that every later LDS read might alias (it would then wait for the
// load before each read and no copy could overlap the work on earlier
// tiles).  lds_base must be the same in every lane.  The caller orders it:
// s_waitcnt vmcnt, then a barrier, before any wave reads the destination.
// m0 is written here and declared clobbered; the kernels that use this keep
// nothing else in m0.
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(src)
                 : "memory", "m0");
}
// The same copy addressed as a uniform base (an SGPR pair) plus a 32-bit
// per-lane byte offset: the per-lane part stays in one VGPR across copies,
// and a new base costs scalar instructions only.
__device__ __forceinline__ void lds_dma16_sv(const void *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)p;
}

// The softmax floor of Ops.SoftmaxRow (exp(max(x - max, -80)),
// Ops.cs:231,245,256) in base-2 units.
constexpr float kFloor2 = -80.0f * 1.4426950408889634f;

}  // namespace hymt
