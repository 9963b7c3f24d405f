// The KIVI packed mode of the dense decode-attention kernel (dense_kernel.hpp): the reference's kivi_decode_attention
// (attention/kivi.py:199-309, kernel attention/_kivi_kernels.py:14-326) over a KIVIPacked record, i.e. the dense
// kernel's split-K attention with a different load: for row b the first keys_quantized[b] keys and the first
// values_quantized[b] values come from their packed codes (2, 4 or 8 bits, any key and value group), fp16 scales and
// zero points, code * scale + zero in fp32 rounded to the K/V format, and every later slot from the dense buffers or
// the rings. The split plan, the tile order and the arithmetic are the dense kernel's, so the result is bit-identical
// to the dense kernel over buffers that hold the dequantized values (the reference's own test of its kernel,
// tests/unit/test_attention_kivi.py:1-7).

#include "dense_kernel.hpp"

namespace eco {

namespace {

template <int DP, int FMT>
int launch_packed(const DenseParams& p, hipStream_t stream) {
    if constexpr (DP > 256 && FMT == FP32) {
        return fail("kivi decode: fp32 keys and values take head dims up to 256 (bf16 or fp16 ones up to 512)");
    } else {
        const int programs = p.batch * p.kv_heads * p.m_tiles;
        const int slices = DP > 256 ? (p.value_dim + 255) / 256 : 1;  // value slices of 256 channels
        if (p.mask)
            hipLaunchKernelGGL((dense_split_kernel<DP, FMT, FMT, true, 0, true>), dim3(programs, p.splits, slices),
                               dim3(64), 0, stream, p);
        else
            hipLaunchKernelGGL((dense_split_kernel<DP, FMT, FMT, false, 0, true>), dim3(programs, p.splits, slices),
                               dim3(64), 0, stream, p);
        return check_launch("dense_split_kernel (KIVI packed)");
    }
}

template <int DP>
int packed_by_format(const DenseParams& p, hipStream_t stream) {
    switch (p.q_format) {
        case BF16: return launch_packed<DP, BF16>(p, stream);
        case FP16: return launch_packed<DP, FP16>(p, stream);
        case FP32: return launch_packed<DP, FP32>(p, stream);
        default: return fail("kivi decode: queries must be bf16, fp16 or fp32");
    }
}

}  // namespace

int kivi_packed_attention(const DenseParams& p, int padded_dim, hipStream_t stream) {
    if (p.kv_format != p.q_format) return fail("kivi decode: K/V must be in the query's dtype");
    switch (padded_dim) {
        case 64: return packed_by_format<64>(p, stream);
        case 128: return packed_by_format<128>(p, stream);
        case 256: return packed_by_format<256>(p, stream);
        case 512: return packed_by_format<512>(p, stream);
        default: return fail("kivi decode: head dims above 512 are not supported");
    }
}

}  // namespace eco
