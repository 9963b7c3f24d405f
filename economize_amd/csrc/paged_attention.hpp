// Parameters of the paged decode-attention kernels (paged_attention.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

// Virtual pages of row b: without a page list, its ceil(len / 16) pages; with one (Quest), the n_sel listed pages
// (logical page indices, -1 for none) followed by the dense tail, logical pages done[b] .. ceil(len / 16) - 1.
// Split s of a row covers virtual pages [s * split_pages, (s + 1) * split_pages).
struct PagedParams {
    const uint16_t* q;  // bf16 [B, Q, Hq, D], channel stride 1
    int64_t sq_b, sq_q, sq_h;
    const uint8_t* k_cache;  // [pages, Hkv, D / X, 16, X]
    const uint8_t* v_cache;  // [pages, Hkv, D, 16]
    int64_t kc_page, kc_head, vc_page, vc_head;  // byte strides
    const int32_t* block_table;  // [B, bt_cols] with row stride bt_stride
    int64_t bt_stride;
    int bt_cols, num_pages;
    const int32_t* seq_lens;  // tokens of every row (the queries' own included)
    const int32_t* page_list;  // optional [B, Hkv, n_sel]
    int64_t pl_b, pl_h;
    int n_sel;
    const int32_t* done;  // [B] first page of the dense tail (with a page list)
    const float* k_scale;  // optional [Hkv]
    const float* v_scale;
    const float* sinks;  // optional [Hq] logits
    int32_t* counters;  // [B * Hkv], zero between calls (the merging split resets its counter)
    float* part_o;
    float* part_m;
    float* part_l;
    uint16_t* out;  // bf16 [B, Q, Hq, D], channel stride 1
    int64_t so_b, so_q, so_h;
    int batch, queries, q_heads, kv_heads, groups, rows, head_dim, kv_format;
    int split_pages, max_splits;
    int fused;  // 1: merge in the last split of each row; 0: write partials only (profiling)
    float scale, softcap;
};

int paged_split(const PagedParams& p, hipStream_t stream);

}  // namespace eco
