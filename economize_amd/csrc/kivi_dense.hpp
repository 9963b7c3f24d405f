// Parameters of KIVI's in-place fake quantization of dense K/V buffers (kivi_dense.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eco {

struct KiviFakeParams {
    void* buf;                 // [B, H, S, D], channel stride 1, element format `format` (bf16, fp16, fp32)
    int format;
    int64_t sb, sh, ss;        // element strides
    int batch, heads, head_dim;
    int start, stop;           // slots [start, stop) of every row
    int bits, group;           // keys: tokens per group ((stop - start) % group == 0); values: channels per group
    int keys;                  // 1: per channel over token groups; 0: per token over channel groups
};

int kivi_fake_quantize(const KiviFakeParams& p, hipStream_t stream);

}  // namespace eco
