// Parameters of the KIVI kernels (kivi.hip): the quantization schedule, the residual ring, quantize-and-append into
// 32-token pages, and decode attention over the pages and the ring.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

// Byte offsets of one (page, KV head) block of the paged KIVI cache (32 tokens, key groups of 32 tokens, value
// groups of 32 channels): key codes [32][D * bits / 8], value codes (words, see kivi.hip), key scales [D], key zero
// points [D], value scales [D / 32][32], value zero points [D / 32][32] (fp16).
struct KiviLayout {
    int head_dim, bits;
    __host__ __device__ constexpr int codes() const { return 32 * head_dim * bits / 8; }
    __host__ __device__ constexpr int k_codes() const { return 0; }
    __host__ __device__ constexpr int v_codes() const { return codes(); }
    __host__ __device__ constexpr int k_scale() const { return 2 * codes(); }
    __host__ __device__ constexpr int k_zero() const { return k_scale() + 2 * head_dim; }
    __host__ __device__ constexpr int v_scale() const { return k_zero() + 2 * head_dim; }
    __host__ __device__ constexpr int v_zero() const { return v_scale() + 2 * head_dim; }
    __host__ __device__ constexpr int size() const { return v_zero() + 2 * head_dim; }
};

struct KiviParams {
    static constexpr int kPage = 32;  // tokens per cache page
    static constexpr int kTile = 1;   // cache pages per tile
    static constexpr bool kPageList = false;
    const uint16_t* q;  // bf16 [B, Q, Hq, D], channel stride 1
    int64_t sq_b, sq_q, sq_h;
    const uint8_t* blocks;  // [pages, Hkv, block bytes]
    int64_t blk_page, blk_head;
    const uint16_t* k_ring;  // bf16 [B, Hkv, W, D]
    const uint16_t* v_ring;  // bf16 [B, Hkv, D, W]
    int ring;
    const int32_t* keys_quantized;    // [B]
    const int32_t* values_quantized;  // [B]
    const int32_t* block_table;
    int64_t bt_stride;
    int bt_cols, num_pages;
    const int32_t* seq_lens;
    const float* sinks;
    const uint32_t* mask;  // optional packed mask (stream_k.hpp mask_word): visible = causal limit and mask bit
    int64_t mk_b, mk_h, mk_q;
    int mask_words;
    int32_t* counters;
    float* part;
    uint16_t* out;
    int64_t so_b, so_q, so_h;
    int batch, queries, q_heads, kv_heads, groups, rows, head_dim, bits;
    int queries_after;  // queries of the call after this launch's (a call cut in query chunks): they shift the causal limit
    int grid;
    float scale, softcap;
};

struct KiviQuantParams {
    const void* src;  // token t of row b, head h, channel d at b * ss_b + h * ss_h + slot * ss_t + d * ss_d
    int src_format;
    int64_t ss_b, ss_h, ss_t, ss_d;
    int src_start, src_ring;  // slot = t - src_start, or t % src_ring with a ring
    const int32_t* from;      // [B] first token to quantize
    const int32_t* to;        // [B] end of the tokens to quantize
    uint8_t* blocks;
    int64_t blk_page, blk_head;
    const int32_t* block_table;
    int64_t bt_stride;
    int bt_cols, num_pages;
    int batch, kv_heads, head_dim, bits;
    uint32_t* overflow;  // optional: set to 1 when a scale or zero point is beyond fp16
};

struct KiviRingParams {
    const void* k_new;  // [T, Hkv, D] element strides sk_t, sk_h (channel stride 1)
    const void* v_new;
    int in_format;
    int64_t sk_t, sk_h, sv_t, sv_h;
    const int32_t* rows;       // [T] batch row of every token
    const int32_t* positions;  // [T] position of every token in its row (< 0: skip)
    int tokens;
    uint16_t* k_ring;
    uint16_t* v_ring;
    int batch, kv_heads, head_dim, ring;
};

int kivi_schedule(const int32_t* committed, int residual, int32_t* keys_quantized, int32_t* values_quantized,
                  int32_t* ranges, int batch, hipStream_t stream);
int kivi_ring_write(const KiviRingParams& p, hipStream_t stream);
int kivi_quantize(const KiviQuantParams& p, int kind, int max_tokens, hipStream_t stream);
int kivi_resident_groups(int head_dim, int bits, int rows, int* per_cu, int* waves);  // workgroups per CU, waves per workgroup
int kivi_attention(const KiviParams& p, hipStream_t stream);
// The attention of more than 32 query rows per KV head over two-page tiles (kivi_verify.hip).
int kivi_verify_resident_groups(int head_dim, int bits, int* per_cu);
int kivi_verify_attention(const KiviParams& p, hipStream_t stream);

}  // namespace eco
