// Parameters of the dense decode-attention kernels (dense_attention.hip): a few queries per row over K/V buffers
// [B, Hkv, S, D] with any element strides (channel stride 1) and an optional boolean mask.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

struct DenseParams {
    const void* q;  // [B, Hq, Q, D], element strides sq_*, format q_format (bf16, fp16, fp32)
    int64_t sq_b, sq_h, sq_q;
    int q_format;
    const void* k;  // [B, Hkv, S, D], format kv_format (q_format, or fp8 e4m3 / e5m2)
    const void* v;  // [B, Hkv, S, Dv]
    int kv_format;
    int64_t sk_b, sk_h, sk_s, sv_b, sv_h, sv_s;
    const float* k_scale;  // [Hkv] or null (fp8 only)
    const float* v_scale;
    const uint8_t* mask;  // bool [B, Hq, Q, S] through strides (0 = broadcast), or null: every key visible
    int64_t sm_b, sm_h, sm_q, sm_s;
    const float* sinks;  // [Hq] or null
    void* out;           // [B, Q, Hq, Dv], element strides so_*, format q_format
    int64_t so_b, so_q, so_h;
    int32_t* counters;  // [programs]: splits finished (zero when a call starts; the last split leaves it zero)
    float* part;        // [programs][splits][16 rows][2 + padded Dv]: max, sum, accumulators
    int batch, queries, q_heads, kv_heads, groups, rows, keys, head_dim, value_dim;
    int m_tiles, splits;  // blocks of 16 query rows; split s takes the 32-key tiles s, s + splits, ...
    float scale, softcap;
    // Gathered mode (gk non-null; the reference's gathered_decode_attention, attention/gathered.py:96-179): `keys` is
    // the virtual key axis. Virtual key t of (b, kvh) is compact entry t of gk / gv [B, Hkv, capacity, D] below
    // count[b, kvh] (its mask column index[b, kvh, t]), else dense slot start[b] + t - count[b, kvh] of k / v, whose
    // slots number dense_keys. Counts are clamped to the capacity, starts to [0, dense_keys], mask columns to the
    // slots, so that malformed counts read wrong entries but nothing outside the buffers.
    const void* gk;
    const void* gv;
    int64_t sgk_b, sgk_h, sgk_s, sgv_b, sgv_h, sgv_s;
    const int32_t* g_index;  // [B, Hkv, capacity] with strides sgi_b, sgi_h (contiguous entries)
    int64_t sgi_b, sgi_h;
    const int32_t* g_count;  // [B * Hkv]
    const int32_t* g_start;  // [B]
    int g_capacity, dense_keys;
    // Cells mode (cells non-null; the reference's paged_kivi_attention over vLLM's cells, backends/vllm/kivi/
    // kernels.py:216-415): key t of row b and KV head kvh is the dense K entry of the cell at byte
    // block_table[b, t / page_size] * sc_page + kvh * sc_head + (t % page_size) * sc_token, its value cell_off_v bytes
    // further; row b has seq_lens[b] keys. Page ids outside [0, num_pages) are clamped (wrong results, no access
    // outside the cache).
    const uint8_t* cells;
    int64_t sc_page, sc_head, sc_token;
    int page_size, num_pages, cell_off_v;
    const int32_t* block_table;
    int64_t bt_stride;
    int bt_cols;
    const int32_t* seq_lens;
    // Cells read through their codes (code_bits 2 or 4; bf16 cells of 128 channels, key groups of 32 tokens, eight
    // key-aux slots per cell): a key or value whose cell flag is 1 is dequantized from the cell's codes (byte offsets
    // cell_off_kc / cell_off_vc, channels packed along the bytes), its value scales and zero points (cell_off_vs: the
    // token's fp16 scales, then its zero points) and its group's key scales and zero points (cell_off_ka: entry e of
    // the group's 2 D in the cell of the group's token e / 8), as the reference's kernel does; any other flag reads
    // the dense entry. code_bits 0: every key and value from its dense entry.
    int code_bits, cell_off_vs, cell_off_ka, cell_off_kc, cell_off_vc, cell_off_flag;
    // Varlen queries (query_start_loc non-null): query row qi of row b is token query_start_loc[b] + qi (strides sq_q,
    // so_q; sq_b, so_b unused), rows qi >= that row's query count are inactive. causal: key t is visible to query row
    // qi when t < keys_b - queries_b + qi + 1 (on top of the mask).
    const int32_t* query_start_loc;
    int causal;
    // Quest mode (qp_list non-null; the reference's quest_decode_attention over a dense cache, attention/quest.py:
    // 239-344 and _quest_kernels.py:13-97): virtual key t of (b, kvh) is slot qp_list[b, kvh, t >> qp_shift] *
    // 2^qp_shift + t % 2^qp_shift of k / v while t < count (the page size times the list's non-negative entries,
    // which lead it: pages in increasing order, then -1), else slot qp_done[b] * 2^qp_shift + t - count; `keys` bounds
    // the virtual axis and dense_keys the slots. Entries and done are clamped to the buffer's whole pages, so a
    // malformed list reads wrong slots but nothing outside the buffers.
    const int32_t* qp_list;
    int64_t sqp_b, sqp_h;
    int qp_pages, qp_shift;
    const int32_t* qp_done;
    // KIVI packed mode (kp_kc non-null; the reference's kivi_decode_attention over a KIVIPacked record,
    // attention/kivi.py:80-309): key t of (b, kvh) below kp_kq[b] is code * scale + zero of its codes (bits per
    // channel, channel d in byte d * bits / 8 at bit (d % (8 / bits)) * bits) and of its key group's fp16 scales and
    // zero points (group t / kp_kg), value t below kp_vq[b] likewise with its own scales and zero points (channel
    // group d / kp_vg), computed in fp32 and rounded to the K/V format; every other key or value is read from k / v,
    // at slot t, or at slot t % kp_ring of the rings k / v when kp_ring > 0. Counts are clamped to [0, keys].
    const uint8_t* kp_kc;  // key codes [B, Hkv, S, D * bits / 8], byte strides skc_*
    int64_t skc_b, skc_h, skc_s;
    const uint16_t* kp_ks;  // key scales [B, Hkv, ceil(S / kp_kg), D] (fp16 bits), element strides sks_*
    const uint16_t* kp_kz;  // key zero points, in the scales' layout
    int64_t sks_b, sks_h, sks_g;
    const uint8_t* kp_vc;  // value codes [B, Hkv, S, Dv * bits / 8], byte strides svc_*
    int64_t svc_b, svc_h, svc_s;
    const uint16_t* kp_vs;  // value scales [B, Hkv, S, Dv / kp_vg] (fp16 bits), element strides svs_*
    const uint16_t* kp_vz;  // value zero points, in the scales' layout
    int64_t svs_b, svs_h, svs_s;
    const int32_t* kp_kq;  // [B]
    const int32_t* kp_vq;  // [B]
    int kp_bits, kp_kg, kp_vg, kp_ring;
};

int dense_padded_dim(int head_dim, int value_dim);  // 64, 128, 256 or 512; 0 when none fits
int dense_attention(const DenseParams& p, int padded_dim, hipStream_t stream);
// The KIVI packed mode (kp_kc set): bf16, fp16 or fp32 queries with K/V in the query's format (kivi_packed.hip).
int kivi_packed_attention(const DenseParams& p, int padded_dim, hipStream_t stream);

}  // namespace eco
