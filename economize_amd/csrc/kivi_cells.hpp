// Parameters of KIVI on vLLM's paged cell layout (kivi_cells.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

// One cell per (page, KV head, token): [K: D | V: D | value scales: nvg fp16 | value zeros: nvg fp16 |
// key aux: ka fp16 | key codes: D / pb bytes | value codes: D / pb bytes | key flag | value flag], 16-byte aligned.
struct CellLayout {
    int head_dim, element_size, bits, group, value_group, key_aux;
    int off_v, off_vs, off_vz, off_ka, off_kc, off_vc, off_flag, size;
};

struct CellsParams {
    uint8_t* cache;                 // [pages, Hkv, page_size] cells, byte strides sb, sh, sn
    int64_t sb, sh, sn;
    int format;                     // the dense entries' dtype: bf16, fp16 or fp32
    int page_size, num_pages;
    const int32_t* block_table;     // [requests, bt_cols], row stride bt_stride
    int64_t bt_stride;
    int bt_cols;
    const int32_t* query_start_loc;  // [requests + 1]
    const int32_t* seq_lens;         // [requests], tokens after the pass
    const int32_t* prefilling;       // [requests], nonzero: prompt not done (nothing quantized)
    int requests, kv_heads, residual;
    CellLayout L;
};

// plan: device scratch of 4 int32 per (request, KV head)
int kivi_cells_quantize(const CellsParams& p, int32_t* plan, hipStream_t stream);
int kivi_cells_clear_flags(const CellsParams& p, const int32_t* slots, int tokens, hipStream_t stream);

}  // namespace eco
