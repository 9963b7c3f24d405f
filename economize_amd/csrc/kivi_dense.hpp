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

// KIVI's packed record (the reference's KIVIPacked layout, attention/kivi.py:80-132) written from a dense buffer or a
// ring: slots [from[b], to[b]) of every row of src [B, H, slots, D] (slot s at s % src_ring with a ring), keys (per
// channel over `group` tokens; from and to multiples of group) or values (per token over `group` channels, group
// dividing D), their codes into codes [B, H, S, D * bits / 8] (byte strides sc_*), their fp16 scales and zero points
// into scale / zero (element strides sz_*; keys [B, H, ceil(S / group), D] at row s / group, values [B, H, S,
// D / group]); write_back: the source elements replaced by code * scale + low rounded to the source's format.
struct KiviPackParams {
    void* src;
    int format;
    int64_t ss_b, ss_h, ss_s;  // element strides
    int src_ring, write_back;
    uint8_t* codes;
    int64_t sc_b, sc_h, sc_s;
    uint16_t* scale;
    uint16_t* zero;
    int64_t sz_b, sz_h, sz_s;
    const int32_t* from;
    const int32_t* to;
    int batch, heads, head_dim, bits, group, max_tokens, keys;
    int slots;           // slots of the record (and of src without a ring): ranges are clamped to them
    uint32_t* overflow;  // or null: set to 1 when a scale or zero point lies beyond fp16
};

int kivi_pack_quantize(const KiviPackParams& p, hipStream_t stream);

// The dense view of one kind of a packed record: out[b, h, s, d] (s < slots) is code * scale + zero rounded to the
// output format where s < quantized[b], else the full-precision entry at slot s % ring_slots of `ring` (slot s when
// ring_slots is 0).
struct KiviRecordGatherParams {
    const uint8_t* codes;
    int64_t sc_b, sc_h, sc_s;
    const uint16_t* scale;
    const uint16_t* zero;
    int64_t sz_b, sz_h, sz_s;
    const int32_t* quantized;
    const void* ring;
    int64_t sr_b, sr_h, sr_s;
    int ring_slots;
    void* out;
    int format;  // of the ring and the output
    int64_t so_b, so_h, so_s;
    int batch, heads, slots, head_dim, bits, group, keys;
};

int kivi_packed_gather(const KiviRecordGatherParams& p, hipStream_t stream);

}  // namespace eco
