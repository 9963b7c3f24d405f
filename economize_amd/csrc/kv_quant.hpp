// Parameters of the paged append and scale kernels (kv_quant.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

struct AppendParams {
    const void* k_new;  // [T, Hkv, D], channel stride 1, element format in_format
    const void* v_new;
    int in_format;
    int64_t sk_t, sk_h, sv_t, sv_h;  // element strides
    const int32_t* slots;  // [T], slot = page * 16 + position, < 0: skip
    int tokens;
    uint8_t* k_cache;
    uint8_t* v_cache;
    int64_t kc_page, kc_head, vc_page, vc_head;  // byte strides
    int kv_heads, head_dim, num_pages, cache_format;
    const float* k_scale;  // optional [Hkv] (fp8 caches)
    const float* v_scale;
};

struct AbsmaxParams {
    const void* x;  // [A, H, S, D] with element strides
    int in_format;
    int a, h, s, d;
    int64_t sa, sh, ss, sd;
    uint32_t* absmax_bits;  // [H], max-accumulated (zero it first)
};

int paged_append(const AppendParams& p, hipStream_t stream);
int head_absmax(const AbsmaxParams& p, hipStream_t stream);
int scales_from_absmax(const uint32_t* absmax_bits, int heads, int format, float* scales, hipStream_t stream);

}  // namespace eco
