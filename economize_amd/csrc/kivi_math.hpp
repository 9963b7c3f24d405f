// The arithmetic of the reference's KIVI quantize (techniques/kv_quant/kivi.py:121-140) for one group, shared by the
// paged quantize kernels (kivi.hip) and the in-place fake quantization of dense buffers (kivi_dense.hip): low and
// high are the group's fp32 minimum and maximum; scale = fp16r((high - low) / levels) and low = fp16r(low), fp16r
// rounding to fp16 (nearest even) where |x| <= 65504 and keeping x otherwise; code = round_half_even((x - low) /
// safe) clamped to [0, levels], safe = scale where it is positive, else 1. Both divisions are IEEE divisions.
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

}  // namespace eco
