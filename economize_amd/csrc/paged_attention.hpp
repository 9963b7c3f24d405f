// Parameters of the paged decode-attention kernel (paged_attention.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

// Virtual pages of row b: without a page list, its ceil(len / 16) pages; with one (Quest), the span cache pages of
// each of the n_sel listed pages (listed page e covers logical cache pages e * span .. e * span + span - 1; -1 for
// none), followed by the dense tail, logical cache pages done[b] * span .. ceil(len / 16) - 1.
struct PagedParams {
    static constexpr int kPage = 16;   // tokens per cache page
    static constexpr int kTile = 4;    // cache pages per tile
    static constexpr bool kPageList = true;
    const uint16_t* q;  // bf16 [B, Q, Hq, D], channel stride 1 (fp16 with an fp8 cache when out_f16 is set)
    int64_t sq_b, sq_q, sq_h;
    const uint8_t* k_cache;  // [pages, Hkv, D / X, 16, X]
    const uint8_t* v_cache;  // [pages, Hkv, D, 16]
    int64_t kc_page, kc_head, vc_page, vc_head;  // byte strides
    const int32_t* block_table;  // [B, bt_cols] with row stride bt_stride
    int64_t bt_stride;
    int bt_cols, num_pages;
    const int32_t* seq_lens;  // tokens of every row (the queries' own included)
    const int32_t* page_list;  // optional [B, Hkv, n_sel] listed pages of span cache pages each
    int64_t pl_b, pl_h;
    int n_sel, span;
    const int32_t* done;  // [B] first listed-size page of the dense tail (with a page list)
    const float* k_scale;  // optional [Hkv]
    const float* v_scale;
    const float* sinks;  // optional [Hq] logits
    const uint32_t* mask;  // optional packed mask (stream_k.hpp mask_word): visible = causal limit and mask bit
    int64_t mk_b, mk_h, mk_q;
    int mask_words;
    int32_t* counters;  // [B * Hkv], zero between calls (the merging wave resets its row's counter)
    float* part;        // [2 * grid, rows, D + 2]: per workgroup two slots of a row segment's maxima, sums, accumulators
    uint16_t* out;  // bf16 [B, Q, Hq, D], channel stride 1 (fp16 when out_f16 is set)
    int out_f16;    // fp16 queries and output (an fp8 cache only)
    int64_t so_b, so_q, so_h;
    int batch, queries, q_heads, kv_heads, groups, rows, head_dim, kv_format;
    int queries_after;  // queries of the call after this launch's (a call cut in query chunks): they shift the causal limit
    int grid;  // workgroups launched
    float scale, softcap;
};

// Resident workgroups per CU of the kernel instance for this shape, and its waves per workgroup.
int paged_resident_groups(int head_dim, int format, int rows, int* per_cu, int* waves);
int paged_attention(const PagedParams& p, hipStream_t stream);
// The same with fp16 queries and output (fp8 caches, whole rows: no page list; paged_attention_f16.hip).
int paged_resident_groups_f16(int head_dim, int format, int rows, int* per_cu, int* waves);
int paged_attention_f16(const PagedParams& p, hipStream_t stream);

}  // namespace eco
