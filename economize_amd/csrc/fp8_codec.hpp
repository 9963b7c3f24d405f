// Bit-level float conversions shared by the kernels and the host: bf16 rounding and the fp8 encoder.
// Written without HIP headers so that the same code compiles for the CPU (its CPU test compiles it with g++).
#pragma once

#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define ECO_HD __host__ __device__
#else
#define ECO_HD
#endif

namespace eco {

// ---- bit helpers --------------------------------------------------------------------------------------------
ECO_HD inline uint32_t f32_bits(float x) {
    union { float f; uint32_t u; } c;
    c.f = x;
    return c.u;
}

ECO_HD inline float bits_f32(uint32_t u) {
    union { float f; uint32_t u; } c;
    c.u = u;
    return c.f;
}

ECO_HD inline float bf16_to_f32(uint16_t h) { return bits_f32(static_cast<uint32_t>(h) << 16); }

// float32 -> bf16 bits, round to nearest even (NaN kept quiet).
ECO_HD inline uint16_t f32_to_bf16(float x) {
    uint32_t u = f32_bits(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
    return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// float32 inside the format's finite range -> fp8 byte, round to nearest even (the OCP cast that
// torch.Tensor.to(float8_e4m3fn / float8_e5m2) performs after the reference's clamp). Normal values round the
// float32 mantissa on its bit pattern; subnormal ones are multiples of the smallest subnormal, which a power-of-two
// scaling and rintf (round half to even) give exactly.
template <int FMT>  // 1 = e4m3fn, 2 = e5m2 (the Format codes of common.hpp)
ECO_HD inline uint8_t f32_to_fp8(float x) {
    constexpr int MB = FMT == 1 ? 3 : 2;          // mantissa bits
    constexpr int BIAS = FMT == 1 ? 7 : 15;
    constexpr uint32_t MIN_NORMAL = static_cast<uint32_t>(127 + 1 - BIAS) << 23;
    constexpr float SUB_SCALE = FMT == 1 ? 512.0f : 65536.0f;  // 1 / smallest subnormal
    uint32_t u = f32_bits(x);
    uint32_t sign = (u >> 24) & 0x80u;
    u &= 0x7FFFFFFFu;
    if (u > 0x7F800000u) return static_cast<uint8_t>(sign | 0x7Fu);
    if (u >= MIN_NORMAL) {
        constexpr int DROP = 23 - MB;
        uint32_t r = (u + ((1u << (DROP - 1)) - 1u) + ((u >> DROP) & 1u)) >> DROP;
        return static_cast<uint8_t>(sign | (r - (static_cast<uint32_t>(127 - BIAS) << MB)));
    }
    float m = rintf(bits_f32(u) * SUB_SCALE);
    return static_cast<uint8_t>(sign | static_cast<uint32_t>(m));
}

}  // namespace eco
