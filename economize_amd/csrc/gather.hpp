// Parameters of the dense views of the paged caches (gather.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

struct PagedGatherParams {
    const uint8_t* k_cache;  // [pages, Hkv, D / X, 16, X]
    const uint8_t* v_cache;  // [pages, Hkv, D, 16]
    int64_t kc_page, kc_head, vc_page, vc_head;  // byte strides
    int kv_format;
    const float* k_scale;  // optional [Hkv]
    const float* v_scale;
    const int32_t* block_table;
    int64_t bt_stride;
    int bt_cols, num_pages;
    void* k_out;  // [B, Hkv, keys, D], element strides so_k*, format out_format
    void* v_out;
    int64_t so_kb, so_kh, so_ks, so_vb, so_vh, so_vs;
    int out_format;
    int batch, kv_heads, keys, head_dim;
};

struct KiviGatherParams {
    const uint8_t* blocks;  // [pages, Hkv, block bytes]
    int64_t blk_page, blk_head;
    const uint16_t* k_ring;  // bf16 [B, Hkv, W, D]
    const uint16_t* v_ring;  // bf16 [B, Hkv, D, W]
    int ring;
    const int32_t* keys_quantized;
    const int32_t* values_quantized;
    const int32_t* block_table;
    int64_t bt_stride;
    int bt_cols, num_pages;
    void* k_out;
    void* v_out;
    int64_t so_kb, so_kh, so_ks, so_vb, so_vh, so_vs;
    int out_format;
    int batch, kv_heads, keys, head_dim, bits;
};

int paged_gather(const PagedGatherParams& p, hipStream_t stream);
int kivi_gather(const KiviGatherParams& p, hipStream_t stream);

}  // namespace eco
