// Shared definitions of the economize_amd HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <string>

#include "fp8_codec.hpp"

namespace eco {

// Element formats of the C-ABI (economize_amd.h).
enum Format : int { BF16 = 0, FP8_E4M3 = 1, FP8_E5M2 = 2, FP16 = 3, FP32 = 4 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// ---- errors -------------------------------------------------------------------------------------------------
void set_error(const std::string& message);
int fail(const std::string& message);  // set_error + return 1
int check_launch(const char* what);    // 0, or 2 with the HIP error of the last launch recorded

template <int FMT>
ECO_HD constexpr float fp8_max() {
    return FMT == FP8_E4M3 ? 448.0f : 57344.0f;
}

// The larger of a and b, NaN if either is NaN (v_maximum_f32 / v_maximum3_f32). Unlike fmaxf it needs no quieting
// of its operands, which the compiler otherwise inserts wherever it cannot prove an operand is not a signalling NaN.
__device__ inline float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ inline float group_max(float x) {  // max over the four lanes l, l^16, l^32, l^48 (NaN if any is NaN)
    x = max_nan(x, __shfl_xor(x, 16));
    return max_nan(x, __shfl_xor(x, 32));
}

__device__ inline float group_sum(float x) {  // sum over the four lanes l, l^16, l^32, l^48
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

// Device-coherent (agent-scope) store and load of partial results handed between workgroups (gfx950 lowers them to
// global_store / global_load with sc1: written through to, and read from, the level every XCD sees). The kernels order
// a hand-off with signal fences, a wait for the stores' completion and an agent-scope counter.
__device__ inline void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline float coherent_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// cap * tanh(x / cap) in log2 units (times log2 e), with inv_cap = 1 / cap: tanh(|t|) = (1 - e) / (1 + e), e =
// exp(-2 |t|), through the hardware exp2 and reciprocal (each within a few ulp; the reference's soft cap is the same
// expression in fp32).
__device__ inline float soft_cap_log2(float x, float cap, float inv_cap) {
    const float t = x * inv_cap;
    const float e = __builtin_amdgcn_exp2f(-2.0f * kLog2e * fabsf(t));
    const float th = (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e);
    return cap * kLog2e * (t < 0.0f ? -th : th);
}

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// A 16-byte load of cache data read once per call (K/V tiles, codes): nontemporal, so the line is streamed rather than
// kept in the caches. A load-only copy of the fp8 decode's access pattern (2 KB page blocks through a shuffled table,
// 268 MB per call over three copies) takes 39.6 us this way against 45.8 us with plain loads.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ inline uint4 stream_load16(const void* p) {
    const u32x4_t x = __builtin_nontemporal_load(static_cast<const u32x4_t*>(p));
    return make_uint4(x.x, x.y, x.z, x.w);
}

}  // namespace eco
