// The bounds of one Quest page of the paged key cache, by one wave (shared by the Quest kernels and the append that
// keeps the bounds up to date): the channel-wise smallest and largest stored key over the page's tokens, fp8 decoded
// exactly, written as bf16 (attention/quest.py:54-65).
#pragma once

#include "common.hpp"
#include "quest.hpp"

namespace eco {

template <int FMT>
__device__ inline float quest_decode_elem(const uint8_t* p, int i) {
    if constexpr (FMT == BF16) {
        return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    } else {
        // exact fp8 value, through the hardware converter (scale 1)
        const uint32_t word = p[i];
        if constexpr (FMT == FP8_E4M3)
            return __builtin_amdgcn_cvt_scalef32_f32_fp8(word, 1.0f, 0);
        else
            return __builtin_amdgcn_cvt_scalef32_f32_bf8(word, 1.0f, 0);
    }
}

// The bounds of Quest page qp of (row b, KV head kvh) by one wave: lane l holds token l % 16 of the runs l / 16,
// l / 16 + 4, ... of every cache page of the Quest page; the 16 lanes of a run then reduce over the tokens.
template <int FMT>
__device__ inline void quest_bounds_of_page(const BoundsParams& p, int b, int qp, int kvh, int lane) {
    constexpr int ES = FMT == BF16 ? 2 : 1;
    constexpr int X = 16 / ES;  // channels per 16-byte run
    const int runs = p.head_dim / X;
    const int token = lane & 15;
    // every cache page of the Quest page must be held (a missing one leaves the bounds untouched)
    for (int s = 0; s < p.span; ++s) {
        const int lp = qp * p.span + s;
        if (lp >= p.bt_cols) return;
        const int phys = p.block_table[b * p.bt_stride + lp];
        if (phys < 0 || phys >= p.num_pages) return;
    }
    for (int r0 = 0; r0 < runs; r0 += 4) {
        const int run = r0 + (lane >> 4);
        float lo[X], hi[X];
#pragma unroll
        for (int i = 0; i < X; ++i) {
            lo[i] = INFINITY;
            hi[i] = -INFINITY;
        }
        if (run < runs) {
            for (int s = 0; s < p.span; ++s) {
                const int phys = p.block_table[b * p.bt_stride + qp * p.span + s];
                const uint8_t* src = p.k_cache + static_cast<int64_t>(phys) * p.kc_page + kvh * p.kc_head +
                                     (run * 16 + token) * 16;
                uint8_t raw[16];
                *reinterpret_cast<uint4*>(raw) = *reinterpret_cast<const uint4*>(src);
#pragma unroll
                for (int i = 0; i < X; ++i) {
                    const float v = quest_decode_elem<FMT>(raw, i);
                    lo[i] = fminf(lo[i], v);
                    hi[i] = fmaxf(hi[i], v);
                }
            }
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1)
#pragma unroll
            for (int i = 0; i < X; ++i) {
                lo[i] = fminf(lo[i], __shfl_xor(lo[i], off));
                hi[i] = fmaxf(hi[i], __shfl_xor(hi[i], off));
            }
        if (run < runs && token == 0) {
            const int64_t at = b * p.sb_b + kvh * p.sb_h + qp * p.sb_p + run * X;
#pragma unroll
            for (int i = 0; i < X; ++i) {
                p.kmin[at + i] = f32_to_bf16(lo[i]);
                p.kmax[at + i] = f32_to_bf16(hi[i]);
            }
        }
    }
}

}  // namespace eco
