// The launches of the dense decode-attention kernel (dense_kernel.hpp): the instance for the head dim, the query
// and K/V formats and the mask, in one launch per call.

#include "dense_kernel.hpp"

namespace eco {

namespace {

template <int DP, int FMT, int QF>
int launch_dense(const DenseParams& p, hipStream_t stream) {
    const int programs = p.batch * p.kv_heads * p.m_tiles;
    if constexpr (DP > 256 && FMT == FP32) {
        return fail("decode: fp32 keys and values take head dims up to 256 (bf16, fp16 or fp8 ones up to 512)");
    } else {
    const int slices = DP > 256 ? (p.value_dim + 255) / 256 : 1;  // value slices of 256 channels
    if constexpr (DP == 128 && FMT == BF16 && QF == BF16) {
        if (p.code_bits == 2 && !p.mask) {
            hipLaunchKernelGGL((dense_split_kernel<DP, FMT, QF, false, 2>), dim3(programs, p.splits), dim3(64), 0,
                               stream, p);
            return check_launch("dense_split_kernel");
        }
        if (p.code_bits == 4 && !p.mask) {
            hipLaunchKernelGGL((dense_split_kernel<DP, FMT, QF, false, 4>), dim3(programs, p.splits), dim3(64), 0,
                               stream, p);
            return check_launch("dense_split_kernel");
        }
    }
    if (p.code_bits) return fail("decode: codes are read for bf16 cells of 128 channels without a mask only");
    if (p.mask)
        hipLaunchKernelGGL((dense_split_kernel<DP, FMT, QF, true>), dim3(programs, p.splits, slices), dim3(64), 0,
                           stream, p);
    else
        hipLaunchKernelGGL((dense_split_kernel<DP, FMT, QF, false>), dim3(programs, p.splits, slices), dim3(64), 0,
                           stream, p);
    return check_launch("dense_split_kernel");
    }
}

template <int DP, int QF>
int by_kv_format(const DenseParams& p, hipStream_t stream) {
    switch (p.kv_format) {
        case FP8_E4M3: return launch_dense<DP, FP8_E4M3, QF>(p, stream);
        case FP8_E5M2: return launch_dense<DP, FP8_E5M2, QF>(p, stream);
        default: return launch_dense<DP, QF, QF>(p, stream);  // K/V in the query's format
    }
}

template <int DP>
int by_q_format(const DenseParams& p, hipStream_t stream) {
    switch (p.q_format) {
        case BF16: return by_kv_format<DP, BF16>(p, stream);
        case FP16: return by_kv_format<DP, FP16>(p, stream);
        case FP32: return by_kv_format<DP, FP32>(p, stream);
        default: return fail("decode: queries must be bf16, fp16 or fp32");
    }
}

}  // namespace

int dense_padded_dim(int head_dim, int value_dim) {
    const int d = head_dim > value_dim ? head_dim : value_dim;
    if (d <= 64) return 64;
    if (d <= 128) return 128;
    if (d <= 256) return 256;
    if (d <= 512) return 512;
    return 0;
}

int dense_attention(const DenseParams& p, int padded_dim, hipStream_t stream) {
    switch (padded_dim) {
        case 64: return by_q_format<64>(p, stream);
        case 128: return by_q_format<128>(p, stream);
        case 256: return by_q_format<256>(p, stream);
        case 512: return by_q_format<512>(p, stream);
        default: return fail("decode: head dims above 512 are not supported");
    }
}

}  // namespace eco
