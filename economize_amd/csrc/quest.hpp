// Parameters of the Quest kernels (quest.hip): page bounds over the paged key cache, page scores, top-k selection.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

struct BoundsParams {
    const uint8_t* k_cache;  // [pages, Hkv, D / X, 16, X]
    int64_t kc_page, kc_head;  // byte strides
    int kv_format, num_pages;
    const int32_t* block_table;  // [B, bt_cols], row stride bt_stride
    int64_t bt_stride;
    int bt_cols;
    int first, last;  // Quest pages [first, last) of every row
    int span;         // cache pages (16 tokens) per Quest page
    uint16_t* kmin;   // bf16 [B, Hkv, P, D], element strides
    uint16_t* kmax;
    int64_t sb_b, sb_h, sb_p;
    int batch, kv_heads, head_dim;
    // device-driven refresh (quest_refresh): pages [valid[b * Hkv + h], min(committed[b] / (16 * span), page_cap))
    const int32_t* committed;  // [B] committed tokens
    int32_t* valid;            // [B * Hkv] Quest pages whose bounds are final
    int32_t* done;             // optional [B]: committed Quest pages, written for the selection and the attention
    int page_cap;              // Quest pages the bounds hold
};

struct SelectParams {
    const void* q;  // [B, Q, Hq, D] in q_format (bf16, fp16, fp32), channel stride 1
    int64_t sq_b, sq_q, sq_h;
    int q_format;
    const void* kmin;  // [B, Hkv, P, D] in bounds_format (bf16, fp16, fp32), channel stride 1
    const void* kmax;
    int64_t sb_b, sb_h, sb_p;
    int bounds_format;
    const int32_t* done;  // [B] committed Quest pages of every row
    int max_done, pages;
    int first_page;   // nonzero: a row's page 0 is always selected (it scores +inf)
    int32_t* out;     // [B, Hkv, pages]
    float* scores;    // workspace [B, Hkv, max_done]
    int batch, queries, q_heads, kv_heads, groups, head_dim;
    int chunk;        // pages scored per workgroup
};

// Page bounds over a dense key buffer [B, Hkv, S, D] (the reference's own cache layout).
struct DenseBoundsParams {
    const void* keys;  // format kv_format (bf16, fp16, fp32, fp8 e4m3 / e5m2), element strides sk_*, channel stride 1
    int64_t sk_b, sk_h, sk_s;
    int kv_format;
    int first, last, page;  // pages [first, last) of `page` slots each
    void* kmin;             // [B, Hkv, P, D] in bounds_format, element strides sb_*; page p at p * sb_p
    void* kmax;
    int64_t sb_b, sb_h, sb_p;
    int bounds_format;  // bf16 for bf16 and fp8 keys, else the keys' format
    int batch, kv_heads, head_dim;
};

int quest_bounds(const BoundsParams& p, hipStream_t stream);
int quest_dense_bounds(const DenseBoundsParams& p, hipStream_t stream);
int quest_refresh(const BoundsParams& p, hipStream_t stream);
int quest_select(const SelectParams& p, hipStream_t stream);
int quest_score_chunk(int head_dim);  // pages scored per workgroup

}  // namespace eco
