// The arithmetic of the reference's KIVI quantize (techniques/kv_quant/kivi.py:121-140) for one group, shared by the
// paged quantize kernels (kivi.hip) and the in-place fake quantization of dense buffers (kivi_dense.hip): low and
// high are the group's fp32 minimum and maximum; scale = fp16r((high - low) / levels) and low = fp16r(low), fp16r
// rounding to fp16 (nearest even) where |x| <= 65504 and keeping x otherwise; code = round_half_even((x - low) /
// safe) clamped to [0, levels], safe = scale where it is positive, else 1. Both divisions are IEEE divisions. Also
// the exact conversion of packed codes to fp32 used by the attention kernels (kivi.hip, kivi_verify.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

__device__ inline float fp16_rounded(float x) {
    return fabsf(x) <= 65504.0f ? static_cast<float>(static_cast<_Float16>(x)) : x;
}

struct Quant {
    float scale, low, safe;
};

// overflow (optional): set to 1 when the scale or the zero point stays in fp32 (beyond the fp16 range).
__device__ inline Quant make_quant(float lo, float hi, int levels, uint32_t* overflow) {
    Quant q;
    q.scale = fp16_rounded(__fdiv_rn(hi - lo, static_cast<float>(levels)));
    q.low = fp16_rounded(lo);
    q.safe = q.scale > 0.0f ? q.scale : 1.0f;
    if (overflow && (fabsf(q.scale) > 65504.0f || fabsf(q.low) > 65504.0f)) atomicOr(overflow, 1u);
    return q;
}

__device__ inline uint32_t code_of(float x, const Quant& q, int levels) {
    const float c = rintf(__fdiv_rn(x - q.low, q.safe));
    return static_cast<uint32_t>(fminf(fmaxf(c, 0.0f), static_cast<float>(levels)));
}

// The code as a float, NaN kept (torch's round and clamp propagate NaN).
__device__ inline float code_or_nan(float x, const Quant& q, int levels) {
    const float c = rintf(__fdiv_rn(x - q.low, q.safe));
    return c != c ? c : fminf(fmaxf(c, 0.0f), static_cast<float>(levels));
}

// A code c < 16 zero-extended to a byte is the e4m3 pattern of c * 2^-9, so v_cvt_scalef32_pk_f32_fp8 with scale
// 2^9 gives the exact fp32 value c.
// Eight codes of a word as exact fp32 values, in element order: for 4-bit codes the word's 8 elements, for 2-bit
// codes elements 8 h .. 8 h + 7 of its 16.
template <int BITS>
__device__ inline void codes_to_f32(uint32_t word, int h, float (&out)[8]) {
    uint32_t lo, hi;
    if constexpr (BITS == 4) {
        lo = word & 0x0F0F0F0Fu;
        hi = (word >> 4) & 0x0F0F0F0Fu;
    } else {
        lo = (word >> (4 * h)) & 0x03030303u;
        hi = (word >> (4 * h + 2)) & 0x03030303u;
    }
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, false);
    const f32x2 b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, true);
    const f32x2 c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, false);
    const f32x2 d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, true);
    out[0] = a.x;
    out[1] = a.y;
    out[2] = b.x;
    out[3] = b.y;
    out[4] = c.x;
    out[5] = c.y;
    out[6] = d.x;
    out[7] = d.y;
}

}  // namespace eco
