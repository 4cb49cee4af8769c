// gemv.hip -- y (+)= W x for the reference's quantized weight formats, one
// token (decode): the weight GEMVs of a decode step (HunyuanDenseModel.Decode.cs
// DecodeQkv / DecodeLinear / DecodeGateUp; Vulkan dec_gemvadd_*.comp).
//
// Weights sit in HBM in the device layout of hymt_weight_upload (weights.cpp):
// every format is cut into 32-value units whose bytes are 8- or 16-byte
// aligned, so a lane reads its units with plain vector loads.  HBM-bound: a
// decode GEMV moves 1-15 MB, so the kernel is as much about memory latency as
// bandwidth: a lane issues the loads of all its units before it touches x.
//
// Work split: 256 threads (4 waves).  A row takes a group of LPR lanes (8..64,
// a power of two); lane j of the group handles units j + LPR k (k < K =
// UPR / LPR, UPR = cols / 32 units per row), so neighbouring lanes read
// neighbouring bytes and a row costs one reduction over its group (DPP).  x
// is staged in LDS with the sums of its 8-value runs (the formats' offset
// and min terms need sums of x, not per-value products).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "ktimer.hpp"
#include "weights.hpp"

namespace hymt {
namespace {


// Sum over aligned groups of `lanes` lanes (8, 16, 32 or 64); every lane of
// a group receives it.  DPP within a row of 16 (quad_perm xor 1, xor 2,
// half-row mirror, row mirror), lane shuffles across rows.
__device__ __forceinline__ float group_sum(float v, int lanes) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    if (lanes >= 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    if (lanes >= 32) v += __shfl_xor(v, 16, 64);
    if (lanes >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// bytes 0..3 of w as floats (v_cvt_f32_ubyte0..3)
__device__ __forceinline__ void bytes4(uint32_t w, float *o) {
    o[0] = (float)(w & 0xFFu);
    o[1] = (float)((w >> 8) & 0xFFu);
    o[2] = (float)((w >> 16) & 0xFFu);
    o[3] = (float)(w >> 24);
}

// w & mask with the mask hidden from the optimiser: bytes4 of the result is
// then one v_cvt_f32_ubyteN per byte, where a visible mask would be folded
// into a bit-field extract per byte before each conversion
__device__ __forceinline__ uint32_t masked(uint32_t w, uint32_t mask) {
    uint32_t r = w & mask;
    asm("" : "+v"(r));
    return r;
}

// x is staged in LDS with 4 floats of padding after every 64, so that the
// 16-byte reads of the lanes of a wave (every row of the wave reads the same
// 8 or 16 addresses, 64 floats apart) fall in different banks
__device__ __forceinline__ int xpad(int f) { return f + ((f >> 6) << 2); }

__device__ __forceinline__ float dot4(const float *a, float4 b, float acc) {
    acc = fmaf(a[0], b.x, acc);
    acc = fmaf(a[1], b.y, acc);
    acc = fmaf(a[2], b.z, acc);
    return fmaf(a[3], b.w, acc);
}

// ---- per-format units: load() issues the loads of unit u of row r, dot()
// returns its contribution given x (LDS) and the 8-value sums xs (LDS) ----

struct UnitF32 {
    static constexpr int kMax = 4;  // units in flight per lane
    uint4 v[8];
    __device__ void load(const WeightDev &w, int r, int u) {
        const uint4 *p = (const uint4 *)((const float *)w.q + (size_t)r * w.cols + 32 * u);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = p[i];
    }
    __device__ float dot(const WeightDev &, int, int u, const float *x, const float *) const {
        const float4 *xv = (const float4 *)(x + xpad(32 * u));
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float wv[4] = {__uint_as_float(v[i].x), __uint_as_float(v[i].y), __uint_as_float(v[i].z),
                                 __uint_as_float(v[i].w)};
            a = dot4(wv, xv[i], a);
        }
        return a;
    }
    __device__ void store(int u, float dsc, float *o) const {
#pragma unroll
        for (int i = 0; i < 8; i++)
            *(float4 *)(o + 32 * u + 4 * i) = make_float4(__uint_as_float(v[i].x), __uint_as_float(v[i].y),
                                                          __uint_as_float(v[i].z), __uint_as_float(v[i].w));
    }
};

struct UnitF16 {
    static constexpr int kMax = 4;  // units in flight per lane
    uint4 v[4];
    __device__ void load(const WeightDev &w, int r, int u) {
        const uint4 *p = (const uint4 *)((const uint16_t *)w.q + (size_t)r * w.cols + 32 * u);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = p[i];
    }
    __device__ float dot(const WeightDev &, int, int u, const float *x, const float *) const {
        const float4 *xv = (const float4 *)(x + xpad(32 * u));
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t h[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
            const float w0[4] = {h2f(h[0] & 0xFFFF), h2f(h[0] >> 16), h2f(h[1] & 0xFFFF), h2f(h[1] >> 16)};
            const float w1[4] = {h2f(h[2] & 0xFFFF), h2f(h[2] >> 16), h2f(h[3] & 0xFFFF), h2f(h[3] >> 16)};
            a = dot4(w0, xv[2 * i], a);
            a = dot4(w1, xv[2 * i + 1], a);
        }
        return a;
    }
    __device__ void store(int u, float, float *o) const {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t h[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                o[32 * u + 8 * i + 2 * e] = h2f(h[e] & 0xFFFF);
                o[32 * u + 8 * i + 2 * e + 1] = h2f(h[e] >> 16);
            }
        }
    }
};

// Q8_0 (Q8_0.cs:16-35): q int8 [rows][cols], d fp32 [rows][cols/32]
struct UnitQ8_0 {
    static constexpr int kMax = 8;  // units in flight per lane
    uint4 v[2];
    float d;
    __device__ void load(const WeightDev &w, int r, int u) {
        const uint4 *p = (const uint4 *)((const int8_t *)w.q + (size_t)r * w.cols + 32 * u);
        v[0] = p[0];
        v[1] = p[1];
        d = w.d[(size_t)r * (w.cols / 32) + u];
    }
    __device__ float dot(const WeightDev &, int, int u, const float *x, const float *) const {
        const float4 *xv = (const float4 *)(x + xpad(32 * u));
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t wd = i < 4 ? (&v[0].x)[i] : (&v[1].x)[i - 4];
            const float q[4] = {(float)(int8_t)(wd & 0xFF), (float)(int8_t)((wd >> 8) & 0xFF),
                                (float)(int8_t)((wd >> 16) & 0xFF), (float)(int8_t)(wd >> 24)};
            a = dot4(q, xv[i], a);
        }
        return d * a;
    }
    __device__ void store(int u, float, float *o) const {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t wd = i < 4 ? (&v[0].x)[i] : (&v[1].x)[i - 4];
#pragma unroll
            for (int e = 0; e < 4; e++) o[32 * u + 4 * i + e] = d * (float)(int8_t)((wd >> (8 * e)) & 0xFF);
        }
    }
};

// Q4_K (Q4K.cs:8-19, 36-61): 144-byte super-blocks as stored.  Unit u is
// super-block u/8, sub = u%8 -> g = sub/2, h = sub%2: qs bytes
// 32 g + 16 h + [0,16), their low nibbles at 64 g + 16 h + i (scale 2 g),
// high nibbles at 64 g + 32 + 16 h + i (scale 2 g + 1).
struct UnitQ4_K {
    static constexpr int kMax = 8;  // units in flight per lane
    static constexpr int kGrid = 1024;  // workgroups the lane split aims for (see launch_t)
    uint4 hdr, qs;
    __device__ void load(const WeightDev &w, int r, int u) {
        const uint8_t *b = (const uint8_t *)w.q + ((size_t)r * (w.cols / 256) + (u >> 3)) * 144;
        hdr = *(const uint4 *)b;
        qs = *(const uint4 *)(b + 16 + 16 * (u & 7));
    }
    // scales and mins of sub-blocks 2 g and 2 g + 1 (GetScaleMin, Q4K.cs:8-19);
    // scale bytes s[0..11] are hdr.y, hdr.z, hdr.w, byte k of a dword taken by
    // shift (a run-time index into a register array would go to scratch)
    __device__ void scales(int g, int (&sc)[2], int (&m)[2]) const {
        auto byte = [](uint32_t w, int k) { return (int)((w >> (8 * k)) & 0xFFu); };
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int j = 2 * g + t;
            if (j < 4) {
                sc[t] = byte(hdr.y, j) & 63;
                m[t] = byte(hdr.z, j) & 63;
            } else {
                sc[t] = (byte(hdr.w, j - 4) & 0xF) | ((byte(hdr.y, j - 4) >> 6) << 4);
                m[t] = (byte(hdr.w, j - 4) >> 4) | ((byte(hdr.z, j - 4) >> 6) << 4);
            }
        }
    }
    __device__ float dot(const WeightDev &, int, int u, const float *x, const float *xs) const {
        const int g = (u & 7) >> 1, h = (u & 1);
        const int base = 256 * (u >> 3) + 64 * g + 16 * h;
        const float d = h2f(hdr.x & 0xFFFF), dmin = h2f(hdr.x >> 16);
        int sc[2], m[2];
        scales(g, sc, m);
        const uint32_t wd[4] = {qs.x, qs.y, qs.z, qs.w};
        const float4 *xl = (const float4 *)(x + xpad(base)), *xh = (const float4 *)(x + xpad(base + 32));
        float al = 0.f, ah = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // the high nibbles in place: bytes 16 q, summed then scaled by
            // 1/16 (exact, the sum's roundings scale with it)
            float lo[4], hi[4];
            bytes4(masked(wd[i], 0x0F0F0F0Fu), lo);
            bytes4(masked(wd[i], 0xF0F0F0F0u), hi);
            al = dot4(lo, xl[i], al);
            ah = dot4(hi, xh[i], ah);
        }
        ah *= 0.0625f;
        const float sl = xs[base / 8] + xs[base / 8 + 1], sh = xs[base / 8 + 4] + xs[base / 8 + 5];
        return d * (sc[0] * al + sc[1] * ah) - dmin * (m[0] * sl + m[1] * sh);
    }
    __device__ void store(int u, float, float *o) const {
        const int g = (u & 7) >> 1, h = (u & 1);
        const int base = 256 * (u >> 3) + 64 * g + 16 * h;
        const float d = h2f(hdr.x & 0xFFFF), dmin = h2f(hdr.x >> 16);
        int sc[2], m[2];
        scales(g, sc, m);
        const float d1 = d * sc[0], m1 = dmin * m[0], d2 = d * sc[1], m2 = dmin * m[1];
        const uint32_t wd[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float lo[4], hi[4];
            bytes4(wd[i] & 0x0F0F0F0Fu, lo);
            bytes4((wd[i] >> 4) & 0x0F0F0F0Fu, hi);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                o[base + 4 * i + e] = d1 * lo[e] - m1;
                o[base + 32 + 4 * i + e] = d2 * hi[e] - m2;
            }
        }
    }
};

// Q6_K (Q6K.cs:37-66): 208-byte super-blocks ql[128] qh[64] sc[16], d fp32
// [rows][cols/256].  Unit u: super-block u/8, l8 = u%8 -> half n = l8/4,
// p = l8%4, l = 8 p + i (i < 8): values at 128 n + 32 j + l for j < 4.
struct UnitQ6_K {
    static constexpr int kMax = 8;  // units in flight per lane
    uint2 a, b, h, sc;
    float d;
    __device__ void load(const WeightDev &w, int r, int u) {
        const size_t sb = (size_t)r * (w.cols / 256) + (u >> 3);
        const uint8_t *blk = (const uint8_t *)w.q + sb * 208;
        const int n = (u & 7) >> 2, p = (u & 3);
        a = *(const uint2 *)(blk + 64 * n + 8 * p);
        b = *(const uint2 *)(blk + 64 * n + 32 + 8 * p);
        h = *(const uint2 *)(blk + 128 + 32 * n + 8 * p);
        sc = *(const uint2 *)(blk + 192 + 8 * n);
        d = w.d[sb];
    }
    __device__ float dot(const WeightDev &, int, int u, const float *x, const float *xs) const {
        const int n = (u & 7) >> 2, p = (u & 3);
        const int base = 256 * (u >> 3) + 128 * n + 8 * p;
        // int8 scale i (0..7) of this half: byte i of sc, by shift
        auto scale = [&](int i) { return (float)(int8_t)((((i < 4) ? sc.x : sc.y) >> (8 * (i & 3))) & 0xFFu); };
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int hw = 0; hw < 2; hw++) {  // i = 4 hw + [0, 4)
            const uint32_t A = hw ? a.y : a.x, B = hw ? b.y : b.x, H = hw ? h.y : h.x;
            const uint32_t q1 = (A & 0x0F0F0F0Fu) | ((H & 0x03030303u) << 4);
            const uint32_t q2 = (B & 0x0F0F0F0Fu) | (((H >> 2) & 0x03030303u) << 4);
            const uint32_t q3 = ((A >> 4) & 0x0F0F0F0Fu) | (((H >> 4) & 0x03030303u) << 4);
            const uint32_t q4 = ((B >> 4) & 0x0F0F0F0Fu) | (((H >> 6) & 0x03030303u) << 4);
            uint32_t qq[4] = {q1, q2, q3, q4};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                asm("" : "+v"(qq[j]));  // one v_cvt_f32_ubyteN per code (see masked)
                float f[4];
                bytes4(qq[j], f);
                acc[j] = dot4(f, *(const float4 *)(x + xpad(base + 32 * j + 4 * hw)), acc[j]);
            }
        }
        float a_ = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) a_ += scale(p / 2 + 2 * j) * (acc[j] - 32.f * xs[(base + 32 * j) / 8]);
        return d * a_;
    }
    __device__ void store(int u, float, float *o) const {
        const int n = (u & 7) >> 2, p = (u & 3);
        const int base = 256 * (u >> 3) + 128 * n + 8 * p;
        auto scale = [&](int i) { return (float)(int8_t)((((i < 4) ? sc.x : sc.y) >> (8 * (i & 3))) & 0xFFu); };
#pragma unroll
        for (int hw = 0; hw < 2; hw++) {
            const uint32_t A = hw ? a.y : a.x, B = hw ? b.y : b.x, H = hw ? h.y : h.x;
            const uint32_t qq[4] = {(A & 0x0F0F0F0Fu) | ((H & 0x03030303u) << 4),
                                    (B & 0x0F0F0F0Fu) | (((H >> 2) & 0x03030303u) << 4),
                                    ((A >> 4) & 0x0F0F0F0Fu) | (((H >> 4) & 0x03030303u) << 4),
                                    ((B >> 4) & 0x0F0F0F0Fu) | (((H >> 6) & 0x03030303u) << 4)};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float f[4];
                bytes4(qq[j], f);
                const float ds = d * scale(p / 2 + 2 * j);
#pragma unroll
                for (int e = 0; e < 4; e++) o[base + 32 * j + 4 * hw + e] = ds * (f[e] - 32.f);
            }
        }
    }
};

// Q2_0C (Q2_0C.cs:13-26): codes [rows][cols/4] bytes, d fp32 [rows][cols/512];
// unit u = 8 bytes = values 32 u + [0, 32), value (2 c - 3) d.
struct UnitQ2_0C {
    static constexpr int kMax = 8;  // units in flight per lane
    uint2 q;
    float d;
    __device__ void load(const WeightDev &w, int r, int u) {
        q = *(const uint2 *)((const uint8_t *)w.q + (size_t)r * (w.cols / 4) + 8 * u);
        d = w.d[(size_t)r * (w.cols / 512) + u / 16];
    }
    __device__ float dot(const WeightDev &, int, int u, const float *x, const float *xs) const {
        const float4 *xv = (const float4 *)(x + xpad(32 * u));
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t wd = i ? q.y : q.x;  // 16 codes: byte b holds values 4b + [0,4)
#pragma unroll
            for (int s = 0; s < 4; s++) {
                // value 4 b + s of byte b is bits 2 s of byte b
                float f[4];
                bytes4((wd >> (2 * s)) & 0x03030303u, f);  // codes (4b + s) for b = 0..3
                const float4 x0 = xv[4 * i], x1 = xv[4 * i + 1], x2 = xv[4 * i + 2], x3 = xv[4 * i + 3];
                const float xsel[4] = {(&x0.x)[s], (&x1.x)[s], (&x2.x)[s], (&x3.x)[s]};
                a = fmaf(f[0], xsel[0], a);
                a = fmaf(f[1], xsel[1], a);
                a = fmaf(f[2], xsel[2], a);
                a = fmaf(f[3], xsel[3], a);
            }
        }
        const float sx = xs[4 * u] + xs[4 * u + 1] + xs[4 * u + 2] + xs[4 * u + 3];
        return d * (2.f * a - 3.f * sx);
    }
    __device__ void store(int u, float, float *o) const {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t wd = i ? q.y : q.x;
#pragma unroll
            for (int b = 0; b < 4; b++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    o[32 * u + 16 * i + 4 * b + t] = (float)((int)((wd >> (8 * b + 2 * t)) & 3u) * 2 - 3) * d;
        }
    }
};

// STQ1_0 (STQ1_0.cs:57-101): slots [rows][cols/8] bytes (two per byte), signs
// [rows][cols/32] bytes, d fp32 [rows][cols/256].  Unit u: block u/8, chunk
// c = (u%8)/2, groups 16 c + 8 hg + [0, 8) (hg = u%2): 4 slot bytes, 1 sign
// byte; group gi's lanes are values 64 c + 8 hg + gi + 16 lane.
struct UnitSTQ1_0 {
    static constexpr int kMax = 8;  // units in flight per lane
    uint32_t slots;
    uint32_t signs;
    float d;
    __device__ void load(const WeightDev &w, int r, int u) {
        slots = *(const uint32_t *)((const uint8_t *)w.q + (size_t)r * (w.cols / 8) + 4 * u);
        signs = ((const uint8_t *)w.q2)[(size_t)r * (w.cols / 32) + u];
        d = w.d[(size_t)r * (w.cols / 256) + (u >> 3)];
    }
    __device__ float dot(const WeightDev &, int, int u, const float *x, const float *xs, const uint8_t *book) const {
        const int c = (u & 7) >> 1, hg = (u & 1);
        const int base = 256 * (u >> 3) + 64 * c + 8 * hg;
        uint32_t pk[8];
#pragma unroll
        for (int gi = 0; gi < 8; gi++) pk[gi] = book[(((signs >> gi) & 1) << 4) | ((slots >> (4 * gi)) & 0xF)];
        float a = 0.f;
#pragma unroll
        for (int ln = 0; ln < 4; ln++) {
            const float4 xa = *(const float4 *)(x + xpad(base + 16 * ln)), xb = *(const float4 *)(x + xpad(base + 16 * ln + 4));
            const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int gi = 0; gi < 8; gi++) a = fmaf((float)((pk[gi] >> (2 * ln)) & 3), xv[gi], a);
        }
        const float sx = xs[base / 8] + xs[base / 8 + 2] + xs[base / 8 + 4] + xs[base / 8 + 6];
        return d * (a - sx);
    }
    __device__ void store(int u, const uint8_t *book, float *o) const {
        const int c = (u & 7) >> 1, hg = (u & 1);
        const int base = 256 * (u >> 3) + 64 * c + 8 * hg;
#pragma unroll
        for (int gi = 0; gi < 8; gi++) {
            const uint32_t pk = book[(((signs >> gi) & 1) << 4) | ((slots >> (4 * gi)) & 0xF)];
#pragma unroll
            for (int ln = 0; ln < 4; ln++) o[base + gi + 16 * ln] = (float)((int)((pk >> (2 * ln)) & 3u) - 1) * d;
        }
    }
};

// STQ1_0.Codebook (STQ1_0.cs:57-63)
__constant__ uint8_t kStqBook[32] = {
    0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42,
    0x01, 0x21, 0x81, 0xA1, 0x04, 0x24, 0x84, 0xA4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68,
};

// K = cols / 32 / lpr units per lane and the input mode are template
// arguments: the loads then sit in straight-line code, so the wait before the
// activations' arithmetic counts only the activation loads (a run-time loop
// bound and mode made the compiler wait for every weight load there too, and
// the RMSNorm, the LDS staging and its barriers ran after the weights had
// landed: 0.7 us on the 12288 x 2048 gate/up GEMV).
// MODE is the input mode: 0 x as given, 1 RMSNorm (kGemvInRmsNorm), 2
// SwiGLU (kGemvInSwiGLU); each loads only the vectors it needs.
template <typename Unit, bool STQ, int NJ, int K, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(WeightDev w, const float *__restrict__ xg, float *__restrict__ y,
                                                   int lpr, int flags, const float *__restrict__ nw, float eps) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float *x = smem;                        // [cols + cols / 16] (xpad)
    float *xs = smem + w.cols + w.cols / 16;  // [cols / 8]
    __shared__ uint8_t book[32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // lane group gi computes row gi; with kGemvOutSwiGLU (W = [gate; up], F
    // rows each) the groups alternate gate row gi/2 and up row F + gi/2, so
    // that a row pair sits in neighbouring groups
    const int gi = (blockIdx.x * 4 + wave) * (64 / lpr) + lane / lpr;
    const bool out_swiglu = flags & kGemvOutSwiGLU;
    const int row = out_swiglu ? (gi & 1) * (w.rows >> 1) + (gi >> 1) : gi;
    const int sub = lane % lpr;
    // unit sub + lpr k, written with lpr = 8 lpr8 (lpr is 8, 16, 32 or 64) so
    // that the compiler sees u & 7 = sub & 7: the unit's place inside its
    // 256-value block (and the scale bytes it needs) is a lane constant
    const int lpr8 = lpr >> 3;

    // 1. the activations first (small, from L2: their data returns while the
    // weight loads below are still in flight), then this lane's weight loads,
    // all issued before anything waits.  Thread tid holds the 8 values
    // [8i, 8i+8) for i = tid + 256j, j < NJ = cols / 2048.
    constexpr int nj = NJ;
    constexpr bool swiglu = MODE == 2, rms = MODE == 1;
    float4 xa[NJ], xb[NJ], ua[NJ], ub[NJ], ga[NJ], gb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int i = tid + 256 * j;
        xa[j] = ((const float4 *)xg)[2 * i];
        xb[j] = ((const float4 *)xg)[2 * i + 1];
        if constexpr (swiglu) {
            ua[j] = ((const float4 *)(xg + w.cols))[2 * i];
            ub[j] = ((const float4 *)(xg + w.cols))[2 * i + 1];
        }
        if constexpr (rms) {
            ga[j] = ((const float4 *)nw)[2 * i];
            gb[j] = ((const float4 *)nw)[2 * i + 1];
        }
    }
    Unit un[K];
    const int rl = gi < w.rows ? row : w.rows - 1;
#pragma unroll
    for (int k = 0; k < K; k++) un[k].load(w, rl, sub + 8 * (lpr8 * k));
    // nothing moves across: left free, the scheduler put the RMSNorm's sum
    // of squares (and with it a wait for x) before the weight loads
    __builtin_amdgcn_sched_barrier(0);
    if (STQ && tid < 32) book[tid] = kStqBook[tid];
    // 2. x as the input mode makes it, into LDS with its 8-value sums
    auto silu_mul = [](float4 g, float4 u) {
        // Ops.SiLUMulRange (Ops.cs:1016-1052): g / (1 + exp(-g)) * u
        return make_float4(g.x / (1.f + expf(-g.x)) * u.x, g.y / (1.f + expf(-g.y)) * u.y,
                           g.z / (1.f + expf(-g.z)) * u.z, g.w / (1.f + expf(-g.w)) * u.w);
    };
    if constexpr (swiglu) {
#pragma unroll
        for (int j = 0; j < NJ; j++)
            if (j < nj) {
                xa[j] = silu_mul(xa[j], ua[j]);
                xb[j] = silu_mul(xb[j], ub[j]);
            }
    }
    if constexpr (rms) {
        // x / sqrt(mean(x^2) + eps) * nw (Ops.RmsNorm, Ops.cs:12-90)
        __shared__ float red[4];
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; j++)
            if (j < nj) {
                const float4 a = xa[j], b = xb[j];
                ss += ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) +
                      ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
            }
        ss = group_sum(ss, 64);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const float rr = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)w.cols + eps);
#pragma unroll
        for (int j = 0; j < NJ; j++)
            if (j < nj) {
                const float4 a = xa[j], b = xb[j], g = ga[j], h = gb[j];
                xa[j] = make_float4(a.x * rr * g.x, a.y * rr * g.y, a.z * rr * g.z, a.w * rr * g.w);
                xb[j] = make_float4(b.x * rr * h.x, b.y * rr * h.y, b.z * rr * h.z, b.w * rr * h.w);
            }
    }
#pragma unroll
    for (int j = 0; j < NJ; j++)
        if (j < nj) {
            const int i = tid + 256 * j;
            const float4 a = xa[j], b = xb[j];
            float4 *xd = (float4 *)(x + xpad(8 * i));
            xd[0] = a;
            xd[1] = b;
            xs[i] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        }
    __syncthreads();
    // 3. dot products, then the row's sum over its lane group
    float part = 0.f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        if constexpr (STQ) part += un[k].dot(w, 0, sub + 8 * (lpr8 * k), x, xs, book);
        else part += un[k].dot(w, 0, sub + 8 * (lpr8 * k), x, xs);
    }
    const float s = group_sum(part, lpr);
    if (out_swiglu) {
        // y[gi/2] = silu(gate) * up (Ops.SiLUMul, Ops.cs:1016-1052; the
        // reference's fused decode gate/up, dec_ffngu.comp:9-11, 292-301): the
        // up sum comes from the neighbouring group, in this wave for lpr < 64,
        // else from the neighbouring wave through LDS
        float u;
        if (lpr < 64) {
            u = __shfl_xor(s, lpr, 64);
        } else {
            __shared__ float pair[4];
            if (lane == 0) pair[wave] = s;
            __syncthreads();
            u = pair[wave ^ 1];
        }
        if (sub == 0 && !(gi & 1) && gi < w.rows) y[gi >> 1] = s / (1.f + expf(-s)) * u;
        return;
    }
    if (sub == 0 && gi < w.rows) y[row] = (flags & kGemvAccumulate) ? y[row] + s : s;
}

// One row of the matrix, dequantized (the embedding lookup,
// HunyuanDenseModel.Embed, HunyuanDenseModel.cs:494-557): a workgroup of 256
// threads, one unit per thread and pass.
template <typename Unit, bool STQ>
__global__ __launch_bounds__(256) void embed_kernel(WeightDev w, int row, float *__restrict__ out) {
    __shared__ uint8_t book[32];
    if (STQ && threadIdx.x < 32) book[threadIdx.x] = kStqBook[threadIdx.x];
    __syncthreads();
    for (int u = threadIdx.x; u < w.cols / 32; u += 256) {
        Unit un;
        un.load(w, row, u);
        if constexpr (STQ) un.store(u, book, out);
        else un.store(u, 0.f, out);
    }
}

const char *gemv_span_name(int type) {
    switch (type) {
    case kW_F32: return "gemv_f32";
    case kW_F16: return "gemv_f16";
    case kW_Q8_0: return "gemv_q8_0";
    case kW_Q4_K: return "gemv_q4_k";
    case kW_Q6_K: return "gemv_q6_k";
    case kW_Q2_0C: return "gemv_q2_0c";
    default: return "gemv_stq1_0";
    }
}

template <typename U, typename = void> struct HasGrid : std::false_type {};
template <typename U> struct HasGrid<U, std::void_t<decltype(U::kGrid)>> : std::true_type {};
template <typename Unit> constexpr int unit_grid() {
    if constexpr (HasGrid<Unit>::value) return Unit::kGrid;
    else return 512;
}

template <typename Unit, bool STQ>
hipError_t launch_t(const WeightDev &w, const float *x, float *y, int flags, const float *nw, float eps,
                    hipStream_t s) {
    const int upr = w.cols / 32;
    // a row's units must fit a wave; a thread stages at most 4 x 8 values of x
    if (w.cols % 2048 != 0 || w.cols > 8192 || upr > Unit::kMax * 64) return hipErrorInvalidValue;
    // lanes per row: the fewest (most units in flight per lane, K <= kMax), but
    // more until the grid has kGrid workgroups (512 unless the unit says
    // otherwise): the dequantising arithmetic is then spread over more waves.
    // Measured on the 32-layer decode step: Q4_K at 1024 (gate|up with 1536
    // workgroups of 2 units a lane) 0.935 -> 0.906 ms against 512; the other
    // formats' gate|up GEMVs are a little slower at 1024.
    int lpr = 8;
    while (upr / lpr > Unit::kMax) lpr *= 2;
    auto blocks = [&](int l) { return (w.rows + 4 * (64 / l) - 1) / (4 * (64 / l)); };
    while (lpr < 64 && blocks(lpr) < unit_grid<Unit>()) lpr *= 2;
    const size_t lds = ((size_t)w.cols + w.cols / 16) * 4 + (size_t)w.cols / 8 * 4;
    const dim3 grid(blocks(lpr));
    KernelSpan span(gemv_span_name(w.type), s, true);
    const int K = upr / lpr;  // 64 NJ / lpr with lpr 8..64: a power of two, or 3 or 6 for NJ = 3
    const int mode = (flags & kGemvInRmsNorm) ? 1 : (flags & kGemvInSwiGLU) ? 2 : 0;
    bool ok = false;
    auto go = [&](auto nj_tag, auto k_tag) {
        constexpr int NJ = decltype(nj_tag)::value, KK = decltype(k_tag)::value;
        if constexpr (KK <= Unit::kMax) {
            if (w.cols / 2048 == NJ && K == KK) {
                if (mode == 1)
                    launch(span, gemv_kernel<Unit, STQ, NJ, KK, 1>, grid, dim3(256), lds, s, w, x, y, lpr, flags, nw,
                           eps);
                else if (mode == 2)
                    launch(span, gemv_kernel<Unit, STQ, NJ, KK, 2>, grid, dim3(256), lds, s, w, x, y, lpr, flags, nw,
                           eps);
                else
                    launch(span, gemv_kernel<Unit, STQ, NJ, KK, 0>, grid, dim3(256), lds, s, w, x, y, lpr, flags, nw,
                           eps);
                ok = true;
            }
        }
    };
    using std::integral_constant;
    go(integral_constant<int, 1>{}, integral_constant<int, 1>{});
    go(integral_constant<int, 1>{}, integral_constant<int, 2>{});
    go(integral_constant<int, 1>{}, integral_constant<int, 4>{});
    go(integral_constant<int, 1>{}, integral_constant<int, 8>{});
    go(integral_constant<int, 2>{}, integral_constant<int, 2>{});
    go(integral_constant<int, 2>{}, integral_constant<int, 4>{});
    go(integral_constant<int, 2>{}, integral_constant<int, 8>{});
    go(integral_constant<int, 3>{}, integral_constant<int, 3>{});
    go(integral_constant<int, 3>{}, integral_constant<int, 6>{});
    go(integral_constant<int, 4>{}, integral_constant<int, 4>{});
    go(integral_constant<int, 4>{}, integral_constant<int, 8>{});
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

// Rows of the matrix, dequantized to fp32: workgroup b writes row
// rows[b] (or row0 + b when rows is null) at out + b * cols.  Embedding of a
// prompt (HunyuanDenseModel.Embed's row loop, HunyuanDenseModel.cs:541-556)
// and the source of the dense copies the prefill GEMMs read.
template <typename Unit, bool STQ>
__global__ __launch_bounds__(256) void rows_kernel(WeightDev w, const int *__restrict__ rows, int row0,
                                                   float *__restrict__ out) {
    __shared__ uint8_t book[32];
    if (STQ && threadIdx.x < 32) book[threadIdx.x] = kStqBook[threadIdx.x];
    __syncthreads();
    const int row = rows ? rows[blockIdx.x] : row0 + (int)blockIdx.x;
    float *o = out + (size_t)blockIdx.x * w.cols;
    for (int u = threadIdx.x; u < w.cols / 32; u += 256) {
        Unit un;
        un.load(w, row, u);
        if constexpr (STQ) un.store(u, book, o);
        else un.store(u, 0.f, o);
    }
}

template <typename Unit, bool STQ>
hipError_t launch_rows_t(const WeightDev &w, const int *rows, int row0, int n, float *out, hipStream_t s) {
    KernelSpan span("weight_rows", s, true);
    launch(span, rows_kernel<Unit, STQ>, dim3(n), dim3(256), 0, s, w, rows, row0, out);
    return hipGetLastError();
}

template <typename Unit, bool STQ>
hipError_t launch_embed_t(const WeightDev &w, int row, float *out, hipStream_t s) {
    KernelSpan span("embed", s, true);
    launch(span, embed_kernel<Unit, STQ>, dim3(1), dim3(256), 0, s, w, row, out);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv(const WeightDev &w, const float *x, float *y, int flags, const float *nw, float eps,
                       hipStream_t s) {
    switch (w.type) {
    case kW_F32: return launch_t<UnitF32, false>(w, x, y, flags, nw, eps, s);
    case kW_F16: return launch_t<UnitF16, false>(w, x, y, flags, nw, eps, s);
    case kW_Q8_0: return launch_t<UnitQ8_0, false>(w, x, y, flags, nw, eps, s);
    case kW_Q4_K: return launch_t<UnitQ4_K, false>(w, x, y, flags, nw, eps, s);
    case kW_Q6_K: return launch_t<UnitQ6_K, false>(w, x, y, flags, nw, eps, s);
    case kW_Q2_0C: return launch_t<UnitQ2_0C, false>(w, x, y, flags, nw, eps, s);
    case kW_STQ1_0: return launch_t<UnitSTQ1_0, true>(w, x, y, flags, nw, eps, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rows(const WeightDev &w, const int *rows, int row0, int n, float *out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    switch (w.type) {
    case kW_F32: return launch_rows_t<UnitF32, false>(w, rows, row0, n, out, s);
    case kW_F16: return launch_rows_t<UnitF16, false>(w, rows, row0, n, out, s);
    case kW_Q8_0: return launch_rows_t<UnitQ8_0, false>(w, rows, row0, n, out, s);
    case kW_Q4_K: return launch_rows_t<UnitQ4_K, false>(w, rows, row0, n, out, s);
    case kW_Q6_K: return launch_rows_t<UnitQ6_K, false>(w, rows, row0, n, out, s);
    case kW_Q2_0C: return launch_rows_t<UnitQ2_0C, false>(w, rows, row0, n, out, s);
    case kW_STQ1_0: return launch_rows_t<UnitSTQ1_0, true>(w, rows, row0, n, out, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_embed(const WeightDev &w, int row, float *out, hipStream_t s) {
    switch (w.type) {
    case kW_F32: return launch_embed_t<UnitF32, false>(w, row, out, s);
    case kW_F16: return launch_embed_t<UnitF16, false>(w, row, out, s);
    case kW_Q8_0: return launch_embed_t<UnitQ8_0, false>(w, row, out, s);
    case kW_Q4_K: return launch_embed_t<UnitQ4_K, false>(w, row, out, s);
    case kW_Q6_K: return launch_embed_t<UnitQ6_K, false>(w, row, out, s);
    case kW_Q2_0C: return launch_embed_t<UnitQ2_0C, false>(w, row, out, s);
    case kW_STQ1_0: return launch_embed_t<UnitSTQ1_0, true>(w, row, out, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hymt
