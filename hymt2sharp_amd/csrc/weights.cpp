// weights.cpp -- host repack of GGUF weight rows into the device layout of
// weights.hpp.
#include "weights.hpp"

#include <cstring>

namespace hymt {
namespace {

// HalfBits.ToSingle (BlockLayout.cs:216-245): exact fp16 -> fp32
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

long gguf_row_bytes(int type, int cols) {
    switch (type) {
    case kW_F32: return 4L * cols;
    case kW_F16: return 2L * cols;
    case kW_Q8_0: return cols / 32 * 34L;
    case kW_Q4_K: return cols / 256 * 144L;
    case kW_Q6_K: return cols / 256 * 210L;
    case kW_Q2_0C: return cols / 512 * 130L;
    case kW_STQ1_0: return cols / 256 * 42L;
    default: return -1;
    }
}

bool pack_weight(int type, int rows, int cols, const uint8_t *src, PackedWeight &out) {
    const size_t R = (size_t)rows, C = (size_t)cols;
    const long rb = gguf_row_bytes(type, cols);
    if (rb < 0) return false;
    auto alloc = [&](size_t q, size_t q2, size_t d) {
        out.off_q = 0;
        size_t n = align256(q);
        if (q2) {
            out.off_q2 = n;
            n += align256(q2);
        }
        if (d) {
            out.off_d = n;
            n += align256(d);
        }
        out.buf.assign(n, 0);
    };
    uint8_t *B = nullptr;
    switch (type) {
    case kW_F32:
    case kW_F16:
    case kW_Q4_K:
        alloc(R * rb, 0, 0);
        std::memcpy(out.buf.data(), src, R * rb);
        return true;
    case kW_Q8_0: {  // 34-byte blocks: fp16 d, 32 int8
        alloc(R * C, 0, R * (C / 32) * 4);
        B = out.buf.data();
        float *d = (float *)(B + out.off_d);
        for (size_t b = 0; b < R * (C / 32); b++) {
            const uint8_t *s = src + 34 * b;
            d[b] = half_to_float(rd16(s));
            std::memcpy(B + 32 * b, s + 2, 32);
        }
        return true;
    }
    case kW_Q6_K: {  // 210-byte blocks: ql 128, qh 64, scales 16, fp16 d
        alloc(R * (C / 256) * 208, 0, R * (C / 256) * 4);
        B = out.buf.data();
        float *d = (float *)(B + out.off_d);
        for (size_t b = 0; b < R * (C / 256); b++) {
            const uint8_t *s = src + 210 * b;
            std::memcpy(B + 208 * b, s, 208);
            d[b] = half_to_float(rd16(s + 208));
        }
        return true;
    }
    case kW_Q2_0C: {  // 130-byte blocks: fp16 d, 128 code bytes
        alloc(R * (C / 4), 0, R * (C / 512) * 4);
        B = out.buf.data();
        float *d = (float *)(B + out.off_d);
        for (size_t b = 0; b < R * (C / 512); b++) {
            const uint8_t *s = src + 130 * b;
            d[b] = half_to_float(rd16(s));
            std::memcpy(B + 128 * b, s + 2, 128);
        }
        return true;
    }
    case kW_STQ1_0: {  // 42-byte blocks: 32 slot bytes, 8 sign bytes, fp16 d
        alloc(R * (C / 8), R * (C / 32), R * (C / 256) * 4);
        B = out.buf.data();
        uint8_t *sg = B + out.off_q2;
        float *d = (float *)(B + out.off_d);
        for (size_t b = 0; b < R * (C / 256); b++) {
            const uint8_t *s = src + 42 * b;
            std::memcpy(B + 32 * b, s, 32);
            std::memcpy(sg + 8 * b, s + 32, 8);
            d[b] = half_to_float(rd16(s + 40));
        }
        return true;
    }
    default:
        return false;
    }
}

}  // namespace hymt
