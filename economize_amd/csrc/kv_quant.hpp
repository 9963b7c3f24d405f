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

// fp8 encode of a [B, H, T, D] block into a dense fp8 buffer (both with a contiguous channel axis).
struct EncodeParams {
    const void* src;
    int in_format;
    int64_t ss_b, ss_h, ss_t;  // element strides of the source
    uint8_t* dst;
    int out_format;
    int64_t sd_b, sd_h, sd_t;  // byte strides of the destination
    int batch, heads, tokens, head_dim;
    const float* head_scale;  // optional [H]: one scale per head (the static / per-head modes)
    float* token_scale;       // optional [B, H, T] output: the per-token mode computes and writes its scales
    int64_t st_b, st_h, st_t;
};

int paged_append(const AppendParams& p, hipStream_t stream);
// paged_append plus the Quest refresh of BoundsParams (committed, valid, done, bounds) in one launch; counters: one
// int32 per (row, KV head), zero between calls.
struct BoundsParams;
int paged_append_quest(const AppendParams& p, const BoundsParams& q, int32_t* counters, hipStream_t stream);
int fp8_encode(const EncodeParams& p, hipStream_t stream);
int head_absmax(const AbsmaxParams& p, hipStream_t stream);
int scales_from_absmax(const uint32_t* absmax_bits, int heads, int format, float* scales, hipStream_t stream);

}  // namespace eco
