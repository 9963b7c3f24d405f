// Dense decode attention on CDNA4 matrix cores (gfx950): the reference's decode_attention (attention/decode.py:
// 252-324 and its kernels, attention/_decode_kernels.py:78-226) over K/V buffers [B, Hkv, S, D] / [B, Hkv, S, Dv]
// with any element strides, a boolean mask [B, 1 or Hq, Q or 1, S] (broadcast strides allowed), a soft cap and
// attention sinks. It is what the economize attention function runs for a model cache that keeps dense buffers
// (the fused fp8 cache's fp8 views, bf16 / fp16 / fp32 caches); the paged kernels serve the paged caches.
//
// Definition (attention/decode.py:66-103): out[b, qi, h] = softmax_t(q . k_t * scale, masked) v_t, query head h
// reading KV head h / G, zeros for a query that sees no key, fp32 accumulation. Every product runs on the bf16 MFMA:
// a bf16 or fp8 element is one bf16 operand (exact), an fp16 or fp32 element two (hi = bf16(x), lo = bf16(x - hi);
// exact for fp16, 16 significant bits for fp32), and a product of two-term operands sums hi.hi + hi.lo + lo.hi
// (the lo.lo term is below fp32 rounding of the sum). The softmax weights p are split the same way for P.V. With
// fp16 queries over fp16 or fp8 K/V the products run on the fp16 MFMA instead: one exact product per element pair,
// and p split into fp16 hi + lo.
//
// Work split (flash-decoding, as the reference): the key axis is cut into S splits; one wave takes one (row, KV
// head, block of 16 query rows, split s) and walks the tiles of 32 keys s, s + S, s + 2 S, ... (the block's waves
// read adjacent runs together), the next tile's loads in flight while a tile is computed (two register buffers
// where they fit). The splits of a block combine by log-sum-exp in the last of its waves to finish (an agent-scope
// counter per block in the workspace, left zero by every call), one launch per call; a single split writes its rows
// directly. Per tile, S^T = K Q^T with v_mfma_f32_16x16x32_bf16: A-row m of MFMA block v is key 8 (m / 4) + 4 v +
// m % 4, so that lane (n, g) ends with keys 8 g .. 8 g + 7 of query row n, which is exactly the B operand of
// O^T += V^T P^T; the keys are read token-major from HBM straight into the A operand (16-byte loads).
// V^T needs a lane to hold 8 keys of one channel: the tile's values are staged through LDS (coalesced 16-byte loads,
// rows padded by 16 bytes so that the four lane groups' reads fall in different banks) and read back transposed.

#pragma once

#include <type_traits>

#include "common.hpp"
#include "dense_attention.hpp"

namespace eco {

namespace {

constexpr int TK = 32;  // keys per tile

template <int FMT>
constexpr int elem_bytes() {
    return FMT == FP32 ? 4 : (FMT == BF16 || FMT == FP16 ? 2 : 1);
}

template <int FMT>
constexpr bool two_terms() {
    return FMT == FP16 || FMT == FP32;
}

// Eight consecutive elements of format FMT held in w (16 bytes per word; fp32: two words; fp8: w[0].x, w[0].y), as
// bf16 hi (+ lo for two-term formats).
template <int FMT>
__device__ __forceinline__ void cvt8(const uint4 (&w)[FMT == FP32 ? 2 : 1], bf16x8& hi, bf16x8& lo) {
    if constexpr (FMT == BF16) {
        hi = __builtin_bit_cast(bf16x8, w[0]);
    } else if constexpr (FMT == FP16) {
        const f16x8 x = __builtin_bit_cast(f16x8, w[0]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float f = static_cast<float>(x[i]);
            hi[i] = static_cast<__bf16>(f);
            lo[i] = static_cast<__bf16>(f - static_cast<float>(hi[i]));
        }
    } else if constexpr (FMT == FP32) {
        const float f[8] = {bits_f32(w[0].x), bits_f32(w[0].y), bits_f32(w[0].z), bits_f32(w[0].w),
                            bits_f32(w[1].x), bits_f32(w[1].y), bits_f32(w[1].z), bits_f32(w[1].w)};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hi[i] = static_cast<__bf16>(f[i]);
            lo[i] = static_cast<__bf16>(f[i] - static_cast<float>(hi[i]));
        }
    } else {
        uint4 r;
        if constexpr (FMT == FP8_E4M3) {
            r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0].x, 1.0f, false));
            r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0].x, 1.0f, true));
            r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0].y, 1.0f, false));
            r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0].y, 1.0f, true));
        } else {
            r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w[0].x, 1.0f, false));
            r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w[0].x, 1.0f, true));
            r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w[0].y, 1.0f, false));
            r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w[0].y, 1.0f, true));
        }
        hi = __builtin_bit_cast(bf16x8, r);
    }
}

// The raw words of eight consecutive elements of format FMT at p (16-byte aligned; fp8: 8-byte aligned). The
// 16-byte loads are streamed (stream_load16: bf16 dense decode at B=32 L=4096 112 -> 103 us); fp8's 8-byte loads stay
// plain (streamed, the fp8 views took 78.6 us against 67.2).
template <int FMT>
__device__ __forceinline__ void load8(const uint8_t* p, uint4 (&w)[FMT == FP32 ? 2 : 1]) {
    if constexpr (FMT == FP8_E4M3 || FMT == FP8_E5M2) {
        const uint2 x = *reinterpret_cast<const uint2*>(p);
        w[0] = make_uint4(x.x, x.y, 0, 0);
    } else {
#pragma unroll
        for (int i = 0; i < (FMT == FP32 ? 2 : 1); ++i) w[i] = stream_load16(p + 16 * i);
    }
}

// One element of format FMT as fp32 (exact).
template <int FMT>
__device__ __forceinline__ float elem_f32(const uint8_t* p) {
    if constexpr (FMT == BF16) return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    if constexpr (FMT == FP16) return static_cast<float>(*reinterpret_cast<const _Float16*>(p));
    if constexpr (FMT == FP32) return *reinterpret_cast<const float*>(p);
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const uint32_t w = *p;
    f32x2 r;
    if constexpr (FMT == FP8_E4M3)
        r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
    else
        r = __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(w, 1.0f, false);
    return r.x;
}

// KIVI packed mode: the NB code bytes of a chunk at p (NB-byte aligned), low bytes first.
template <int NB>
__device__ __forceinline__ uint2 load_code_bytes(const uint8_t* p) {
    if constexpr (NB == 8) return *reinterpret_cast<const uint2*>(p);
    else if constexpr (NB == 4) return make_uint2(*reinterpret_cast<const uint32_t*>(p), 0u);
    else if constexpr (NB == 2) return make_uint2(*reinterpret_cast<const uint16_t*>(p), 0u);
    else return make_uint2(*p, 0u);
}

// Code e (BITS wide, element e at bit e BITS of the chunk's bytes) as an exact float.
template <int BITS>
__device__ __forceinline__ float code_f32(uint2 w, int e) {
    const int bit = e * BITS;
    const uint32_t word = bit < 32 ? w.x : w.y;
    return static_cast<float>((word >> (bit & 31)) & ((1u << BITS) - 1u));
}

// The same with the byte count and the code width known at run time only (uniform).
__device__ __forceinline__ uint2 load_code_bytes_rt(int nb, const uint8_t* p) {
    if (nb == 8) return *reinterpret_cast<const uint2*>(p);
    if (nb == 4) return make_uint2(*reinterpret_cast<const uint32_t*>(p), 0u);
    if (nb == 2) return make_uint2(*reinterpret_cast<const uint16_t*>(p), 0u);
    return make_uint2(*p, 0u);
}

__device__ __forceinline__ float code_f32_rt(int bits, uint2 w, int e) {
    const int bit = e * bits;
    const uint32_t word = bit < 32 ? w.x : w.y;
    return static_cast<float>(__builtin_amdgcn_ubfe(word, static_cast<uint32_t>(bit & 31), static_cast<uint32_t>(bits)));
}

// N fp16 values at p (16-byte aligned for 8, 8-byte for 4), as the first N halves of a word.
template <int N>
__device__ __forceinline__ uint4 load_halves(const uint16_t* p) {
    if constexpr (N == 8) {
        return *reinterpret_cast<const uint4*>(p);
    } else {
        const uint2 x = *reinterpret_cast<const uint2*>(p);
        return make_uint4(x.x, x.y, 0u, 0u);
    }
}

__device__ __forceinline__ float half_f32(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// 16 bytes of format FMT from the fp32 values x (rounded to nearest even for bf16 and fp16).
template <int FMT>
__device__ __forceinline__ uint4 pack_chunk(const float (&x)[16 / elem_bytes<FMT>()]) {
    if constexpr (FMT == FP32) {
        return make_uint4(f32_bits(x[0]), f32_bits(x[1]), f32_bits(x[2]), f32_bits(x[3]));
    } else if constexpr (FMT == BF16) {
        bf16x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = static_cast<__bf16>(x[i]);
        return __builtin_bit_cast(uint4, r);
    } else {
        f16x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(x[i]);
        return __builtin_bit_cast(uint4, r);
    }
}

__device__ __forceinline__ void split8(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hi[i] = static_cast<__bf16>(x[i]);
        lo[i] = static_cast<__bf16>(x[i] - static_cast<float>(hi[i]));
    }
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_h(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Eight elements of format FMT (fp16, or fp8 in w[0].x / w[0].y) as fp16, exactly.
template <int FMT>
__device__ __forceinline__ f16x8 to_f16x8(const uint4 (&w)[FMT == FP32 ? 2 : 1]) {
    if constexpr (FMT == FP16) {
        return __builtin_bit_cast(f16x8, w[0]);
    } else {
        static_assert(FMT == FP8_E4M3 || FMT == FP8_E5M2, "fp16 or fp8 elements");
        uint4 r;
        if constexpr (FMT == FP8_E4M3) {
            r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0].x, 1.0f, false));
            r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0].x, 1.0f, true));
            r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0].y, 1.0f, false));
            r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0].y, 1.0f, true));
        } else {
            r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[0].x, 1.0f, false));
            r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[0].x, 1.0f, true));
            r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[0].y, 1.0f, false));
            r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[0].y, 1.0f, true));
        }
        return __builtin_bit_cast(f16x8, r);
    }
}

template <int QF>
__device__ __forceinline__ void load_query8(const DenseParams& p, int64_t offset, bf16x8& hi, bf16x8& lo) {
    uint4 w[QF == FP32 ? 2 : 1];
    load8<QF>(static_cast<const uint8_t*>(p.q) + offset * elem_bytes<QF>(), w);
    cvt8<QF>(w, hi, lo);
}

template <int QF>
__device__ __forceinline__ void store_out(const DenseParams& p, int64_t offset, float x) {
    if constexpr (QF == BF16)
        static_cast<uint16_t*>(p.out)[offset] = f32_to_bf16(x);
    else if constexpr (QF == FP16)
        static_cast<_Float16*>(p.out)[offset] = static_cast<_Float16>(x);
    else
        static_cast<float*>(p.out)[offset] = x;
}

// The output weight of a row whose keys gave maximum m and sum l (log2 units) with the sink logit (-inf: none): the
// accumulators times 2^(m - M), divided by l 2^(m - M) + 2^(sink - M), M = max(m, sink) (decode.py's merge,
// attention/_decode_kernels.py:183-226); 0 where nothing is visible. Returns 2^(m - M) and sets inv = 1 / that sum.
__device__ inline float sink_weight(float m, float l, float sink, float& inv) {
    const float big = fmaxf(m, sink);
    float total = 0.0f, a = 0.0f;
    if (big != -INFINITY) {
        if (m != -INFINITY) {
            a = __builtin_amdgcn_exp2f(m - big);
            total = l * a;
        }
        if (sink != -INFINITY) total += __builtin_amdgcn_exp2f(sink - big);
    }
    inv = total > 0.0f ? 1.0f / total : 0.0f;
    return a;
}

// Eight codes of channels c .. c + 7 packed along bytes (channel c + i at bit i BITS of x), as exact floats. The
// codes are spread one per byte (even channels in lo, odd ones in hi); a code below 16 in a byte is the e4m3 pattern
// of code 2^-9, which v_cvt_scalef32_pk_f32_fp8 with scale 2^9 turns into the exact float, two bytes at a time.
template <int BITS>
__device__ __forceinline__ void cell_codes8(uint32_t x, float (&c)[8]) {
    uint32_t lo, hi;
    if constexpr (BITS == 4) {  // nibbles: channel i at bit 4 i
        lo = x & 0x0F0F0F0Fu;          // channels 0, 2, 4, 6
        hi = (x >> 4) & 0x0F0F0F0Fu;   // channels 1, 3, 5, 7
    } else {  // 2-bit fields of the low 16 bits: channel i at bit 2 i
        const uint32_t u = __builtin_amdgcn_perm(0u, x, 0x0C010C00u);  // bytes: x.byte0, 0, x.byte1, 0
        const uint32_t v = (u | (u << 4)) & 0x0F0F0F0Fu;                // bytes: channels 0-1, 2-3, 4-5, 6-7
        lo = v & 0x03030303u;          // channels 0, 2, 4, 6
        hi = (v >> 2) & 0x03030303u;   // channels 1, 3, 5, 7
    }
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 l0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, false);
    const f32x2 l1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, true);
    const f32x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, false);
    const f32x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, true);
    c[0] = l0.x;
    c[2] = l0.y;
    c[4] = l1.x;
    c[6] = l1.y;
    c[1] = h0.x;
    c[3] = h0.y;
    c[5] = h1.x;
    c[7] = h1.y;
}

// The codes of a chunk (channel i at bit i BITS of its bytes; 8 channels, or the first 4 for fp32 chunks) as exact
// floats: 2- and 4-bit codes through the e4m3 conversion of cell_codes8, 8-bit codes one byte each.
template <int BITS>
__device__ __forceinline__ void chunk_codes(uint2 w, float (&c)[8]) {
    if constexpr (BITS == 8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // (v_cvt_f32_ubyte0..3)
            c[i] = static_cast<float>((w.x >> (8 * i)) & 0xFFu);
            c[4 + i] = static_cast<float>((w.y >> (8 * i)) & 0xFFu);
        }
    } else {
        cell_codes8<BITS>(w.x, c);
    }
}

__device__ __forceinline__ void chunk_codes_rt(int bits, uint2 w, float (&c)[8]) {
    if (bits == 8)
        chunk_codes<8>(w, c);
    else if (bits == 4)
        chunk_codes<4>(w, c);
    else
        chunk_codes<2>(w, c);
}

// bf16(code * scale + zero) of eight channels, the product and the sum in fp32 (one fused multiply-add, the product
// of a code and an fp16 scale being exact), as the reference's _dequant and its .to(DOT_DTYPE).
__device__ __forceinline__ bf16x8 dequant_cell8(const float (&c)[8], const float (&sc)[8], const float (&zr)[8]) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<__bf16>(__builtin_fmaf(c[i], sc[i], zr[i]));
    return r;
}

__device__ __forceinline__ uint32_t word_of(uint4 x, int i) {
    return i == 0 ? x.x : (i == 1 ? x.y : (i == 2 ? x.z : x.w));
}

// CB: 0, or the code bits of a cells instance that reads quantized keys and values through their codes.
// Heads wider than 256 channels (DP = 512; Gemma-4's global layers, attention/decode.py:216-232): a wave computes its
// rows' full scores and accumulates one slice of DV = 256 value channels, slice blockIdx.z (the reference's value
// tiles), at one wave per SIMD; the slices of a block and its splits count on the block's one counter, and the last
// of them merges every channel.
// KP: the KIVI packed mode (DenseParams::kp_*), one tile buffer: every tile's keys and values, read as codes below
// the row's quantized counts and as full-precision entries past them, are dequantized into LDS (a lane turns 16-byte
// chunks of the tile into the K/V format) and the products read both from there. A tile of codes only or of
// full-precision entries only issues its loads in batches of up to 16 chunks; a mixed tile goes chunk by chunk; the
// wave's leading tiles of codes only (D <= 128, no mask) hold the next tile's raw codes in registers while a tile is
// computed (codes_run).
template <int DP, int FMT, int QF, bool MASKED, int CB = 0, bool KP = false>
__global__ __launch_bounds__(64, DP > 256 ? 1 : 2) void dense_split_kernel(DenseParams p) {
    static_assert(CB == 0 || (DP == 128 && FMT == BF16 && QF == BF16 && !MASKED),
                  "codes are read for bf16 cells of 128 channels only");
    static_assert(!KP || (CB == 0 && FMT == QF && (FMT == BF16 || FMT == FP16 || FMT == FP32)),
                  "KIVI codes are read with K/V in the query's format (bf16, fp16 or fp32)");
    constexpr int ES = elem_bytes<FMT>();
    constexpr int DV = DP > 256 ? 256 : DP;  // value channels of a wave
    constexpr int KS = DP / 32;  // k-steps of the S MFMA
    constexpr int ND = DV / 16;  // value blocks of 16 channels
    // fp16 queries over fp16 or fp8 K/V: the products take v_mfma_f32_16x16x32_f16 (every product exact, fp8 being
    // a subset of fp16), one MFMA where bf16 operands need the hi + lo terms of the fp16 elements, and P in fp16
    // hi + lo (22 significant bits) for P.V
    constexpr bool H16 = QF == FP16 && (FMT == FP16 || FMT == FP8_E4M3 || FMT == FP8_E5M2) && CB == 0;
    constexpr bool KLO = two_terms<FMT>() && !H16;
    constexpr bool QLO = two_terms<QF>() && !H16;
    constexpr int ROW = DV * ES + 16;          // LDS bytes per staged value row
    constexpr int CHUNKS = TK * DV * ES / 16;  // 16-byte chunks of a staged value tile (a multiple of 64)
    constexpr int CPR = DV * ES / 16;          // chunks per value row
    constexpr int CPL = CHUNKS / 64;           // chunks per lane
    constexpr bool kStage = CPL <= 8;          // the tile's values pass through registers (loads issued first)
    constexpr int KW = ES == 4 ? 2 : 1;        // 16-byte words of 8 key elements (fp8: the low half of one)
    // The next tile's loads are in flight while a tile is computed (NBUF = 2) when the registers allow: one set of
    // staged values (moved into LDS before the next tile's values are issued into it), two sets of keys (fp8 keys
    // fill half a word; with a mask, eight mask bytes), the accumulators and the query operand within 170 VGPRs
    // (beyond that the second key set spills at two waves per SIMD).
    constexpr int KEY_VGPRS = 2 * KS * KW * (ES == 1 ? 2 : 4) + (MASKED ? 8 : 0);
    constexpr int LIVE_VGPRS = (kStage ? 4 * CPL : 0) + 2 * KEY_VGPRS + 4 * ND + 4 * KS * (QLO ? 2 : 1);
    constexpr int NBUF = KP ? 1 : (CB != 0 || (kStage && LIVE_VGPRS <= 170) ? 2 : 1);
    constexpr int KROW = DP * ES + 16;  // KP: LDS bytes per staged key row
    static_assert(CHUNKS % 64 == 0, "value tiles of whole lane rounds");
    __shared__ __align__(16) uint8_t vtile[TK * ROW];
    __shared__ __align__(16) uint8_t auxl[CB != 0 ? 32 * 16 : 16];  // codes: the tile's key scales and zero points
    __shared__ __align__(16) uint8_t ktile[KP ? TK * KROW : 16];     // KP: the tile's keys

    const int lane = static_cast<int>(threadIdx.x);
    const int n = lane & 15, g = lane >> 4;
    const int prog = blockIdx.x;
    const int split = blockIdx.y;
    const int v0 = static_cast<int>(blockIdx.z) * DV;  // the wave's first value channel
    const int mt = prog % p.m_tiles;
    const int kvh = (prog / p.m_tiles) % p.kv_heads;
    const int b = prog / (p.m_tiles * p.kv_heads);
    const int r = mt * 16 + n;  // the lane's query row (MFMA column n)
    // varlen queries: row b's queries are tokens q_start .. q_start + q_count - 1
    const int q_start = p.query_start_loc ? p.query_start_loc[b] : 0;
    const int q_count = p.query_start_loc ? p.query_start_loc[b + 1] - q_start : p.queries;
    const int gq0 = r < p.rows ? r / p.queries : 0;
    const int qi0 = r < p.rows ? r % p.queries : 0;
    const bool r_ok = r < p.rows && qi0 < q_count;
    const int gq = r_ok ? gq0 : 0;
    const int qi = r_ok ? qi0 : 0;
    const int h = kvh * p.groups + gq;

    // the query operand: row r, channels 32 j + 8 g .. (zero past the head dim and for rows past the group)
    bf16x8 qh[KS], ql[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        const int c = 32 * j + 8 * g;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            qh[j][i] = static_cast<__bf16>(0.0f);
            ql[j][i] = static_cast<__bf16>(0.0f);
        }
        if (r_ok && c < p.head_dim) {
            const int64_t at = b * p.sq_b + h * p.sq_h + static_cast<int64_t>(q_start + qi) * p.sq_q + c;
            if constexpr (H16)  // the fp16 bits themselves are the operand
                qh[j] = __builtin_bit_cast(bf16x8, stream_load16(static_cast<const uint8_t*>(p.q) + at * 2));
            else
                load_query8<QF>(p, at, qh[j], ql[j]);
        }
    }
    const float ks = p.k_scale ? p.k_scale[kvh] : 1.0f;
    const float vs = p.v_scale ? p.v_scale[kvh] : 1.0f;
    const float score_scale = p.softcap > 0.0f ? p.scale * ks : p.scale * ks * kLog2e;
    const float inv_cap = p.softcap > 0.0f ? 1.0f / p.softcap : 0.0f;
    const uint8_t* kbase = static_cast<const uint8_t*>(p.k) + (b * p.sk_b + kvh * p.sk_h) * ES;
    const uint8_t* vbase = static_cast<const uint8_t*>(p.v) + (b * p.sv_b + kvh * p.sv_h) * ES;
    const uint8_t* mrow = MASKED ? p.mask + b * p.sm_b + h * p.sm_h + qi * p.sm_q : nullptr;
    // the key axis: dense slots, or (gathered) the row's compact entries followed by its dense slots from start on,
    // or (cells) the row's seq_lens[b] tokens in its pages
    int count = 0, start = 0, row_keys = p.cells ? min(max(p.seq_lens[b], 0), p.keys) : p.keys;
    const uint8_t* gkbase = kbase;
    const uint8_t* gvbase = vbase;
    const int32_t* gidx = nullptr;
    if (p.gk) {
        count = min(max(p.g_count[b * p.kv_heads + kvh], 0), p.g_capacity);
        start = min(max(p.g_start[b], 0), p.dense_keys);
        row_keys = min(count + p.dense_keys - start, p.keys);
        gkbase = static_cast<const uint8_t*>(p.gk) + (b * p.sgk_b + kvh * p.sgk_h) * ES;
        gvbase = static_cast<const uint8_t*>(p.gv) + (b * p.sgv_b + kvh * p.sgv_h) * ES;
        gidx = p.g_index + b * p.sgi_b + kvh * p.sgi_h;
    }
    // Quest: the row's selected pages (a prefix of its list) come first, then its slots from done[b] pages on
    const int32_t* qlist = nullptr;
    const int page_cap = p.qp_list ? p.dense_keys >> p.qp_shift : 0;  // whole pages in the buffer
    if (p.qp_list) {
        qlist = p.qp_list + b * p.sqp_b + kvh * p.sqp_h;
        int valid = 0;
        for (int i = 0; i < p.qp_pages; i += 64) {
            const int e = i + lane < p.qp_pages ? qlist[i + lane] : -1;
            valid += static_cast<int>(__popcll(__ballot(e >= 0)));
        }
        count = min(valid, page_cap) << p.qp_shift;
        start = min(max(p.qp_done[b], 0), page_cap) << p.qp_shift;
        row_keys = min(count + p.dense_keys - start, p.keys);
    }
    // KIVI packed: the row's quantized counts and its codes, scales and zero points
    int kq = 0, vq = 0;
    const uint8_t *kcb = nullptr, *vcb = nullptr;
    const uint16_t *ksb = nullptr, *kzb = nullptr, *vsb = nullptr, *vzb = nullptr;
    if constexpr (KP) {
        kq = min(max(p.kp_kq[b], 0), p.keys);
        vq = min(max(p.kp_vq[b], 0), p.keys);
        kcb = p.kp_kc + b * p.skc_b + kvh * p.skc_h;
        ksb = p.kp_ks + b * p.sks_b + kvh * p.sks_h;
        kzb = p.kp_kz + b * p.sks_b + kvh * p.sks_h;
        vcb = p.kp_vc + b * p.svc_b + kvh * p.svc_h;
        vsb = p.kp_vs + b * p.svs_b + kvh * p.svs_h;
        vzb = p.kp_vz + b * p.svs_b + kvh * p.svs_h;
    }
    // This wave's tiles interleave with its block's other splits: tile k starts at key (split + k splits) 32, so that
    // the block's waves (one XCD) read adjacent 8 KB runs of the K and V buffers together.
    const int tiles_row = (row_keys + TK - 1) / TK;
    const int my_tiles = split < tiles_row ? (tiles_row - 1 - split) / p.splits + 1 : 0;
    auto tile_start = [&](int k) __attribute__((always_inline)) { return (split + k * p.splits) * TK; };
    // cells: a window over this wave's next 64 tile halves (16 keys each), lane l holding the cache byte offset of
    // the first cell of half win0 + l (its page's cells of this KV head, plus the half's place in the page: a
    // multiple of 16 tokens); a tile reads its halves' offsets from the window (v_readlane) and reloads the window
    // every 32 tiles, so that the tile loads need no block-table load, and no division by the page size, of their
    // own. Quest uses the same window for the slot of each half's first key (page-list entries instead of the
    // block table).
    int win0 = -(1 << 30);
    int64_t win_page = 0;
    auto half_offset = [&](int half) __attribute__((always_inline)) -> int64_t {  // half: uniform
        if (half < win0 || half >= win0 + 64) {
            win0 = half;
            const int mine = half + lane;
            const int first = tile_start(mine >> 1) + (mine & 1) * 16;
            if (p.cells) {
                const int lp = min(first / p.page_size, p.bt_cols - 1);
                const int page =
                    min(max(p.block_table[static_cast<int64_t>(b) * p.bt_stride + lp], 0), p.num_pages - 1);
                win_page = page * p.sc_page + kvh * p.sc_head + static_cast<int64_t>(first % p.page_size) * p.sc_token;
            } else if (first < count) {  // Quest: the slot of the half's first key (a half lies in one page)
                const int e = qlist[min(first >> p.qp_shift, p.qp_pages - 1)];
                win_page = (static_cast<int64_t>(min(max(e, 0), page_cap - 1)) << p.qp_shift) +
                           (first & ((1 << p.qp_shift) - 1));
            } else {
                win_page = start + first - count;
            }
            // wait here for the table load (vmcnt(0)), so that the common path, which reloads nothing, does not
            // wait at the branch's join for every load in flight
            __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        const int at = half - win0;
        const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(win_page), at);
        const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(win_page) >> 32), at);
        return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    };
    // the cache offsets of the first cells of tile k's two 16-key halves (a tile starts at a multiple of 32 keys and
    // pages hold a multiple of 16, so each half lies in one page)
    int64_t cell_h0 = 0, cell_h1 = 0;  // (two variables, not an array: a lane-dependent index of one goes to scratch)
    // (Quest: the slots of the halves' first keys; pages of 32 or more slots, and the tail, keep a tile's halves
    // adjacent)
    auto tile_pages = [&](int k) __attribute__((always_inline)) {
        if (p.cells) {
            cell_h0 = half_offset(2 * k);
            cell_h1 = p.page_size % 32 == 0 ? cell_h0 + 16 * p.sc_token : half_offset(2 * k + 1);
        } else if (p.qp_list) {
            cell_h0 = half_offset(2 * k);
            cell_h1 = p.qp_shift >= 5 ? cell_h0 + 16 : half_offset(2 * k + 1);
        }
    };
    auto quest_slot = [&](int t) __attribute__((always_inline)) -> int64_t {  // t inside the current tile
        return ((t >> 4) & 1 ? cell_h1 : cell_h0) + (t & 15);
    };
    auto cell_row = [&](int t) __attribute__((always_inline)) -> const uint8_t* {  // t inside the current tile
        return p.cells + ((t >> 4) & 1 ? cell_h1 : cell_h0) + static_cast<int64_t>(t & 15) * p.sc_token;
    };
    auto key_row = [&](int t) __attribute__((always_inline)) -> const uint8_t* {
        if constexpr (KP) return kbase + static_cast<int64_t>(p.kp_ring > 0 ? t % p.kp_ring : t) * p.sk_s * ES;
        if (p.cells) return cell_row(t);
        if (p.qp_list) return kbase + quest_slot(t) * p.sk_s * ES;
        return t < count ? gkbase + static_cast<int64_t>(t) * p.sgk_s * ES
                         : kbase + static_cast<int64_t>(start + t - count) * p.sk_s * ES;
    };
    auto value_row = [&](int t) __attribute__((always_inline)) -> const uint8_t* {
        if constexpr (KP) return vbase + static_cast<int64_t>(p.kp_ring > 0 ? t % p.kp_ring : t) * p.sv_s * ES;
        if (p.cells) return cell_row(t) + p.cell_off_v;
        if (p.qp_list) return vbase + quest_slot(t) * p.sv_s * ES;
        return t < count ? gvbase + static_cast<int64_t>(t) * p.sgv_s * ES
                         : vbase + static_cast<int64_t>(start + t - count) * p.sv_s * ES;
    };
    // causal: the last q_count keys of the row are its queries' own tokens
    const int causal_limit = p.causal ? row_keys - q_count + qi + 1 : row_keys;
    auto mask_col = [&](int t) __attribute__((always_inline)) -> int64_t {
        if (p.qp_list) return quest_slot(t);
        return t < count ? min(max(gidx[t], 0), p.dense_keys - 1) : start + t - count;
    };

    float m_i = -INFINITY, l_i = 0.0f;
    f32x4 acc[ND];
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) acc[nd] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int t_end = row_keys;

    // A tile's loads in registers: its values (staged for LDS, one set), its keys (A-row n of S block v is key
    // t0 + 8 (n / 4) + 4 v + n % 4) and, with a mask, the mask bytes of the lane's keys t0 + 8 g + e.
    uint4 vreg[kStage && CB == 0 ? CPL : 1];
    // codes: the lane's value token (t0 + lane / 2, channels 64 (lane % 2) ..): its codes, its scales and zero points
    // and its flags; and the key-aux slot of the tile's cell t0 + lane % 32
    uint4 vcw[CB == 4 ? 2 : 1], vsz, vaux;
    uint32_t vfl = 0;
    struct Keys {
        uint4 k[CB != 0 ? 1 : 2][CB != 0 ? 1 : KS][KW];
        uint32_t m[MASKED ? 8 : 1];
        uint32_t kc[2][CB != 0 ? KS : 1];  // codes: the code word of the lane's channels 32 j + 8 g .. of its key v
        uint32_t kf[2];                    // codes: the flag byte of its key v
        int64_t h0, h1;                    // codes: the tile's half offsets (the next tile's issue moves cell_h*)
    };
    // Every load is issued unconditionally at a clamped address (a key past the split reads the split's last key, a
    // channel past the dims reads channel 0) and what it must not contribute is zeroed where it is used: every path
    // through the loop then issues the same loads, and the wait before a tile's use leaves the younger tile's loads
    // in flight.
    auto issue = [&](Keys& K, int k) __attribute__((always_inline)) {
        const int t0 = tile_start(k);
        tile_pages(k);
        if constexpr (CB != 0) {
            K.h0 = cell_h0;
            K.h1 = cell_h1;
            const uint8_t* vc = cell_row(min(t0 + (lane >> 1), t_end - 1));
#pragma unroll
            for (int i = 0; i < (CB == 4 ? 2 : 1); ++i)
                vcw[i] = *reinterpret_cast<const uint4*>(vc + p.cell_off_vc + 16 * (CB / 2) * (lane & 1) + 16 * i);
            vsz = *reinterpret_cast<const uint4*>(vc + p.cell_off_vs);
            vfl = *(vc + p.cell_off_flag + 1);
            // (every cell of the tile's key group: the tile's 32 cells lie in one page, page_size being a multiple
            // of 32, and a visible key's group aux may sit in a cell past the row's keys)
            vaux = *reinterpret_cast<const uint4*>(cell_row(t0 + (lane & 31)) + p.cell_off_ka);
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const uint8_t* krow = cell_row(min(t0 + 8 * (n >> 2) + 4 * v + (n & 3), t_end - 1));
                K.kf[v] = *(krow + p.cell_off_flag);
#pragma unroll
                for (int j = 0; j < KS; ++j)
                    K.kc[v][j] = *reinterpret_cast<const uint32_t*>(
                        krow + p.cell_off_kc + (CB == 2 ? 4 * (2 * j + (g >> 1)) : 16 * j + 4 * g));
            }
            return;
        }
        if constexpr (MASKED)
#pragma unroll
            for (int e = 0; e < 8; ++e) K.m[e] = mrow[mask_col(min(t0 + 8 * g + e, t_end - 1)) * p.sm_s];
        if constexpr (KP) return;  // (the tile's keys and values are loaded where they are staged)
        if constexpr (kStage)
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int chunk = lane + 64 * i;
                const int t = min(t0 + chunk / CPR, t_end - 1);
                const int c = v0 + (chunk % CPR) * (16 / ES);
                vreg[i] = stream_load16(value_row(t) + (c < p.value_dim ? c : 0) * ES);
            }
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const uint8_t* krow = key_row(min(t0 + 8 * (n >> 2) + 4 * v + (n & 3), t_end - 1));
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const int c = 32 * j + 8 * g;
                load8<FMT>(krow + (c < p.head_dim ? c : 0) * ES, K.k[v][j]);
            }
        }
    };
    // ---- KP: the tile's keys and values into LDS, dequantized where they are codes ----
    // A lane takes 16-byte chunks of CE elements: key chunk i of the tile is key i / KCR, channels (i % KCR) CE ..,
    // value chunk i likewise over the wave's value slice; a chunk past the keys or the dims is zero. Every load of a
    // chunk is issued (its entry, its codes, its scales and zero points); the ones it does not need read the row's
    // first entry instead, a line that stays cached, so that a batch's loads go out together with no branch.
    constexpr int CE = 16 / ES;
    constexpr int KCR = DP / CE;
    constexpr int KCH = TK * KCR / 64;
    constexpr int VCR = DV / CE;
    constexpr int VCH = TK * VCR / 64;
    constexpr int KB = 4;  // key chunks per batch (each holds its entry, codes, scales and zero points)
    constexpr int VB = DP >= 256 || ES == 4 ? 4 : 8;
    auto kp_stage = [&](int t0) __attribute__((always_inline)) {
        const int BITS = p.kp_bits;
        const int NB = CE * BITS / 8;  // code bytes of a chunk
        // A lane's chunks share their channels (KCR and VCR divide 64): key channels kc0 .., value channels vc0 ...
        const int kc0 = (lane % KCR) * CE, vc0 = v0 + (lane % VCR) * CE;
        const bool k_ok = kc0 < p.head_dim, v_ok = vc0 < p.value_dim;
        // ---- a tile of codes only (every key and value quantized, the tile's keys inside one key group, each value
        // chunk inside one value group) or of full-precision entries only: its loads in one batch, or, where the
        // registers would not hold them, in batches of 16 chunks (keys, then values) ----
        constexpr bool ONE_BATCH = KCH + VCH <= 16;
        constexpr int KF = KCH < 16 ? KCH : 16;  // chunks per batch
        constexpr int VF = VCH < 16 ? VCH : 16;
        const int kcc = k_ok ? kc0 : 0, vcc = v_ok ? vc0 : 0;
        uint2 kcw[KF], vcw[VF];
        uint4 ks = make_uint4(0, 0, 0, 0), kz = make_uint4(0, 0, 0, 0);
        uint16_t vs[VF], vz[VF];
        auto codes_keys = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < KF; ++i) {
                const int t = t0 + (lane + 64 * (i0 + i)) / KCR;
                kcw[i] = load_code_bytes_rt(NB, kcb + static_cast<int64_t>(t) * p.skc_s + kcc * BITS / 8);
            }
            const int64_t so = static_cast<int64_t>(t0 / p.kp_kg) * p.sks_g + kcc;
            ks = load_halves<CE>(ksb + so);
            kz = load_halves<CE>(kzb + so);
        };
        auto codes_values = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < VF; ++i) {
                const int t = t0 + (lane + 64 * (i0 + i)) / VCR;
                vcw[i] = load_code_bytes_rt(NB, vcb + static_cast<int64_t>(t) * p.svc_s + vcc * BITS / 8);
                const int64_t so = static_cast<int64_t>(t) * p.svs_s + vcc / p.kp_vg;
                vs[i] = vsb[so];
                vz[i] = vzb[so];
            }
        };
        auto keys_from_codes = [&](int i0) __attribute__((always_inline)) {
            const f16x8 s8 = __builtin_bit_cast(f16x8, ks);
            const f16x8 z8 = __builtin_bit_cast(f16x8, kz);
#pragma unroll
            for (int i = 0; i < KF; ++i) {
                float c[8], x[CE];
                chunk_codes_rt(BITS, kcw[i], c);
#pragma unroll
                for (int e = 0; e < CE; ++e)
                    x[e] = __builtin_fmaf(c[e], static_cast<float>(s8[e]), static_cast<float>(z8[e]));
                *reinterpret_cast<uint4*>(ktile + ((lane + 64 * (i0 + i)) / KCR) * KROW + kc0 * ES) =
                    k_ok ? pack_chunk<FMT>(x) : make_uint4(0, 0, 0, 0);
            }
        };
        auto values_from_codes = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < VF; ++i) {
                const float sc = half_f32(vs[i]), zr = half_f32(vz[i]);
                float c[8], x[CE];
                chunk_codes_rt(BITS, vcw[i], c);
#pragma unroll
                for (int e = 0; e < CE; ++e) x[e] = __builtin_fmaf(c[e], sc, zr);
                *reinterpret_cast<uint4*>(vtile + ((lane + 64 * (i0 + i)) / VCR) * ROW + (vc0 - v0) * ES) =
                    v_ok ? pack_chunk<FMT>(x) : make_uint4(0, 0, 0, 0);
            }
        };
        if (t0 + TK <= kq && t0 + TK <= vq && p.kp_kg % TK == 0 && p.kp_vg % CE == 0) {
            if constexpr (ONE_BATCH) {
                codes_keys(0);
                codes_values(0);
                keys_from_codes(0);
                values_from_codes(0);
            } else {
#pragma nounroll
                for (int i0 = 0; i0 < KCH; i0 += KF) {
                    codes_keys(i0);
                    keys_from_codes(i0);
                }
#pragma nounroll
                for (int i0 = 0; i0 < VCH; i0 += VF) {
                    codes_values(i0);
                    values_from_codes(i0);
                }
            }
            return;
        }
        if (t0 >= kq && t0 >= vq) {
            uint4 kd[KF], vd[VF];
            auto dense_keys = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < KF; ++i) {
                    const int t = min(t0 + (lane + 64 * (i0 + i)) / KCR, t_end - 1);
                    kd[i] = *reinterpret_cast<const uint4*>(key_row(t) + kcc * ES);
                }
            };
            auto dense_values = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < VF; ++i) {
                    const int t = min(t0 + (lane + 64 * (i0 + i)) / VCR, t_end - 1);
                    vd[i] = *reinterpret_cast<const uint4*>(value_row(t) + vcc * ES);
                }
            };
            auto keys_to_lds = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < KF; ++i) {
                    const int tl = (lane + 64 * (i0 + i)) / KCR;
                    *reinterpret_cast<uint4*>(ktile + tl * KROW + kc0 * ES) =
                        k_ok && t0 + tl < t_end ? kd[i] : make_uint4(0, 0, 0, 0);
                }
            };
            auto values_to_lds = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < VF; ++i) {
                    const int tl = (lane + 64 * (i0 + i)) / VCR;
                    *reinterpret_cast<uint4*>(vtile + tl * ROW + (vc0 - v0) * ES) =
                        v_ok && t0 + tl < t_end ? vd[i] : make_uint4(0, 0, 0, 0);
                }
            };
            if constexpr (ONE_BATCH) {
                dense_keys(0);
                dense_values(0);
                keys_to_lds(0);
                values_to_lds(0);
            } else {
#pragma nounroll
                for (int i0 = 0; i0 < KCH; i0 += KF) {
                    dense_keys(i0);
                    keys_to_lds(i0);
                }
#pragma nounroll
                for (int i0 = 0; i0 < VCH; i0 += VF) {
                    dense_values(i0);
                    values_to_lds(i0);
                }
            }
            return;
        }
        // ---- any other tile (the row's boundary tiles, value groups inside a chunk): chunk by chunk ----
#pragma nounroll
        for (int base = 0; base < KCH; base += KB) {
            uint4 dn[KB], sc[KB], zr[KB];
            uint2 cw[KB];
#pragma unroll
            for (int i = 0; i < KB; ++i) {
                const int chunk = lane + 64 * (base + i);
                const int t = t0 + chunk / KCR, c = (chunk % KCR) * CE;
                const bool ok = t < t_end && c < p.head_dim;
                const bool code = ok && t < kq;
                const int tt = ok ? t : 0, cc = ok ? c : 0;
                dn[i] = *reinterpret_cast<const uint4*>((code ? kbase : key_row(tt)) + cc * ES);
                cw[i] = load_code_bytes_rt(NB, kcb + (code ? static_cast<int64_t>(tt) * p.skc_s + cc * BITS / 8 : 0));
                const int64_t so = code ? static_cast<int64_t>(tt / p.kp_kg) * p.sks_g + cc : 0;
                sc[i] = load_halves<CE>(ksb + so);
                zr[i] = load_halves<CE>(kzb + so);
            }
#pragma unroll
            for (int i = 0; i < KB; ++i) {
                const int chunk = lane + 64 * (base + i);
                const int tl = chunk / KCR, c = (chunk % KCR) * CE;
                const bool ok = t0 + tl < t_end && c < p.head_dim;
                const bool code = ok && t0 + tl < kq;
                const f16x8 s8 = __builtin_bit_cast(f16x8, sc[i]);
                const f16x8 z8 = __builtin_bit_cast(f16x8, zr[i]);
                float x[CE];
#pragma unroll
                for (int e = 0; e < CE; ++e)
                    x[e] = __builtin_fmaf(code_f32_rt(BITS, cw[i], e), static_cast<float>(s8[e]),
                                          static_cast<float>(z8[e]));
                *reinterpret_cast<uint4*>(ktile + tl * KROW + c * ES) =
                    code ? pack_chunk<FMT>(x) : (ok ? dn[i] : make_uint4(0, 0, 0, 0));
            }
        }
        // values: WHOLE when every chunk lies in one value group (kp_vg a multiple of CE), else a group per element
        auto values = [&](auto whole_c) __attribute__((always_inline)) {
            constexpr bool WHOLE = decltype(whole_c)::value;
            constexpr int NS = WHOLE ? 1 : CE;
            constexpr int B = WHOLE ? VB : 2;  // (a scale and a zero point per element: fewer chunks at once)
#pragma nounroll
            for (int base = 0; base < VCH; base += B) {
                uint4 dn[B];
                uint2 cw[B];
                uint16_t sc[B][NS], zr[B][NS];
#pragma unroll
                for (int i = 0; i < B; ++i) {
                    const int chunk = lane + 64 * (base + i);
                    const int t = t0 + chunk / VCR, c = v0 + (chunk % VCR) * CE;
                    const bool ok = t < t_end && c < p.value_dim;
                    const bool code = ok && t < vq;
                    const int tt = ok ? t : 0, cc = ok ? c : 0;
                    dn[i] = *reinterpret_cast<const uint4*>((code ? vbase : value_row(tt)) + cc * ES);
                    cw[i] = load_code_bytes_rt(NB, vcb + (code ? static_cast<int64_t>(tt) * p.svc_s + cc * BITS / 8 : 0));
                    const int64_t row = code ? static_cast<int64_t>(tt) * p.svs_s : 0;
#pragma unroll
                    for (int e = 0; e < NS; ++e) {
                        const int gi = code ? (cc + e) / p.kp_vg : 0;
                        sc[i][e] = vsb[row + gi];
                        zr[i][e] = vzb[row + gi];
                    }
                }
#pragma unroll
                for (int i = 0; i < B; ++i) {
                    const int chunk = lane + 64 * (base + i);
                    const int tl = chunk / VCR, cl = (chunk % VCR) * CE;
                    const bool ok = t0 + tl < t_end && v0 + cl < p.value_dim;
                    const bool code = ok && t0 + tl < vq;
                    float x[CE];
#pragma unroll
                    for (int e = 0; e < CE; ++e)
                        x[e] = __builtin_fmaf(code_f32_rt(BITS, cw[i], e), half_f32(sc[i][WHOLE ? 0 : e]),
                                              half_f32(zr[i][WHOLE ? 0 : e]));
                    *reinterpret_cast<uint4*>(vtile + tl * ROW + cl * ES) =
                        code ? pack_chunk<FMT>(x) : (ok ? dn[i] : make_uint4(0, 0, 0, 0));
                }
            }
        };
        if (p.kp_vg % CE == 0)
            values(std::true_type{});
        else
            values(std::false_type{});
    };
    // ---- the tile's values into LDS (zero past the keys and past Dv); the previous tile's reads of LDS came first ----
    auto stage = [&](int t0) __attribute__((always_inline)) {
        if constexpr (KP) {
            kp_stage(t0);
            return;
        }
        if constexpr (CB != 0) {
            if (lane < 32) *reinterpret_cast<uint4*>(auxl + 16 * lane) = vaux;
            const int tl = lane >> 1, hh = lane & 1;
            const int t = t0 + tl;
            const bool vok = t < t_end;
            const f16x8 sz = __builtin_bit_cast(f16x8, vsz);  // the token's scales [4] then zero points [4]
            uint4 out[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {  // channels 64 hh + 8 q .., value group 2 hh + q / 4
                // (selects, not an index by the lane's half: a vector indexed at run time goes to scratch)
                const float sc = static_cast<float>(hh ? sz[2 + q / 4] : sz[q / 4]);
                const float zr = static_cast<float>(hh ? sz[6 + q / 4] : sz[4 + q / 4]);
                const uint32_t x = CB == 2 ? (word_of(vcw[0], q >> 1) >> (16 * (q & 1))) & 0xFFFFu
                                           : word_of(vcw[CB == 4 ? (q >> 2) : 0], q & 3);
                float c[8], scs[8], zrs[8];
                cell_codes8<CB>(x, c);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    scs[i] = sc;
                    zrs[i] = zr;
                }
                out[q] = __builtin_bit_cast(uint4, dequant_cell8(c, scs, zrs));
            }
            uint8_t* dst = vtile + tl * ROW + 128 * hh;
            const bool dense = vok && vfl != 1u;  // a cell not quantized: its dense entry
            if (__ballot(dense) != 0) {  // (the loads and their uses stay inside this rare branch)
                if (dense) {
                    const uint8_t* row = cell_row(t) + p.cell_off_v + 128 * hh;
#pragma unroll
                    for (int q = 0; q < 8; ++q) out[q] = *reinterpret_cast<const uint4*>(row + 16 * q);
                }
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    *reinterpret_cast<uint4*>(dst + 16 * q) = vok ? out[q] : make_uint4(0, 0, 0, 0);
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    *reinterpret_cast<uint4*>(dst + 16 * q) = vok ? out[q] : make_uint4(0, 0, 0, 0);
            }
            return;
        }
        if constexpr (kStage) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int chunk = lane + 64 * i;
                const bool ok = t0 + chunk / CPR < t_end && v0 + (chunk % CPR) * (16 / ES) < p.value_dim;
                *reinterpret_cast<uint4*>(vtile + (chunk / CPR) * ROW + (chunk % CPR) * 16) =
                    ok ? vreg[i] : make_uint4(0, 0, 0, 0);
            }
        } else {
            for (int chunk = lane; chunk < CHUNKS; chunk += 64) {
                const int t = chunk / CPR;
                const int c = (chunk % CPR) * (16 / ES);
                uint4 x = make_uint4(0, 0, 0, 0);
                if (t0 + t < t_end && v0 + c < p.value_dim)
                    x = *reinterpret_cast<const uint4*>(value_row(t0 + t) + (v0 + c) * ES);
                *reinterpret_cast<uint4*>(vtile + t * ROW + (chunk % CPR) * 16) = x;
            }
        }
    };
    auto compute = [&](const Keys& K, int t0) __attribute__((always_inline)) {
        // ---- S^T = K Q^T (key channels past the head dim zeroed) ----
        f32x4 s[2];
        if constexpr (CB != 0) {
            // the lane's key scales and zero points (channels 32 j + 8 g ..: entries of the group's aux in the slots
            // of cells 4 j + g and 16 + 4 j + g), then the keys from their codes, or their dense entries where the
            // flag is not 1 (a rare branch that keeps its loads and their uses to itself)
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the aux stores of this tile (one wave: in order)
            auto scores = [&](bool dense) __attribute__((always_inline)) {
#pragma unroll
                for (int v = 0; v < 2; ++v) s[v] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < KS; ++j) {
                    const f16x8 sj = *reinterpret_cast<const f16x8*>(auxl + 16 * (4 * j + g));
                    const f16x8 zj = *reinterpret_cast<const f16x8*>(auxl + 16 * (16 + 4 * j + g));
#pragma unroll
                    for (int v = 0; v < 2; ++v) {
                        const uint32_t x = CB == 2 ? (K.kc[v][j] >> (16 * (g & 1))) & 0xFFFFu : K.kc[v][j];
                        float c[8];
                        cell_codes8<CB>(x, c);
                        bf16x8 kh;  // (the fp16 scales widened inside each product: v_fma_mix_f32)
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            kh[i] = static_cast<__bf16>(
                                __builtin_fmaf(c[i], static_cast<float>(sj[i]), static_cast<float>(zj[i])));
                        if (dense && K.kf[v] != 1u) {
                            const int tk = min(t0 + 8 * (n >> 2) + 4 * v + (n & 3), t_end - 1);
                            const uint8_t* row = p.cells + ((tk >> 4) & 1 ? K.h1 : K.h0) +
                                                 static_cast<int64_t>(tk & 15) * p.sc_token;
                            kh = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(row + 2 * (32 * j + 8 * g)));
                        }
                        s[v] = mfma(kh, qh[j], s[v]);
                    }
                }
            };
            if (__ballot(K.kf[0] != 1u || K.kf[1] != 1u) != 0)
                scores(true);
            else
                scores(false);
        } else {
        if constexpr (KP) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tile's key stores
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            s[v] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                uint4 w[KW];
                const bool ok = 32 * j + 8 * g < p.head_dim;
                if constexpr (KP) {  // key 8 (n / 4) + 4 v + n % 4 of the tile, from LDS
                    const uint8_t* src = ktile + (8 * (n >> 2) + 4 * v + (n & 3)) * KROW + (32 * j + 8 * g) * ES;
#pragma unroll
                    for (int x = 0; x < KW; ++x)
                        w[x] = ok ? *reinterpret_cast<const uint4*>(src + 16 * x) : make_uint4(0, 0, 0, 0);
                } else {
#pragma unroll
                    for (int x = 0; x < KW; ++x) w[x] = ok ? K.k[v][j][x] : make_uint4(0, 0, 0, 0);
                }
                if constexpr (H16) {
                    s[v] = mfma_h(to_f16x8<FMT>(w), __builtin_bit_cast(f16x8, qh[j]), s[v]);
                    continue;
                }
                bf16x8 kh, kl;
                cvt8<FMT>(w, kh, kl);
                s[v] = mfma(kh, qh[j], s[v]);
                if constexpr (QLO) s[v] = mfma(kh, ql[j], s[v]);
                if constexpr (KLO) s[v] = mfma(kl, qh[j], s[v]);
            }
        }
        }
        // ---- scores in log2 units, masked: lane (n, g) holds keys t0 + 8 g + 4 v + i of row r ----
        uint32_t vis = 0;  // bit 4 v + i
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int t = t0 + 8 * g + e;
            bool ok = r_ok && t < t_end && t < causal_limit;
            if constexpr (MASKED) ok = ok && (K.m[e] & 0xFFu) != 0;
            vis |= ok ? 1u << e : 0u;
        }
        float tile_max = -INFINITY;
        // the soft cap tested once per tile, not per score (the compiler keeps a uniform test inside an unrolled loop)
        if (p.softcap > 0.0f) {
#pragma unroll
            for (int v = 0; v < 2; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[v][i] = soft_cap_log2(s[v][i] * score_scale, p.softcap, inv_cap);
        } else {
#pragma unroll
            for (int v = 0; v < 2; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[v][i] *= score_scale;
        }
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x = (vis >> (4 * v + i)) & 1u ? s[v][i] : -INFINITY;
                s[v][i] = x;
                tile_max = max_nan(tile_max, x);
            }
        // ---- online softmax, lazy rescaling (the reference maximum moves when a score exceeds it by 2^8) ----
        if (__ballot(tile_max > m_i + 8.0f || m_i == -INFINITY) != 0) {
            const bool fresh = m_i == -INFINITY;
            const float m_new = fmaxf(m_i, group_max(tile_max));
            const float alpha = fresh ? 0.0f : __builtin_amdgcn_exp2f(m_i - m_new);
            l_i *= alpha;
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[nd][i] = fresh ? 0.0f : acc[nd][i] * alpha;
            m_i = m_new;
        }
        const float neg_m = m_i == -INFINITY ? 0.0f : -m_i;
        float pw[8];
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pw[4 * v + i] = __builtin_amdgcn_exp2f(s[v][i] + neg_m);
                l_i += pw[4 * v + i];
            }
        bf16x8 ph, pl;
        f16x8 ph16, pl16;
        if constexpr (H16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ph16[i] = static_cast<_Float16>(pw[i]);
                pl16[i] = static_cast<_Float16>(pw[i] - static_cast<float>(ph16[i]));
            }
        } else {
            split8(pw, ph, pl);
        }
        // ---- O^T += V^T P^T: lane (n, g) supplies channel 16 nd + n of keys 8 g .. 8 g + 7 ----
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tile's LDS stores (one wave: in order)
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) {
            const int c = 16 * nd + n;  // (of the wave's slice)
            if (v0 + 16 * nd >= p.value_dim) break;
            if constexpr (H16) {
                f16x8 vh16;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if constexpr (FMT == FP16)
                        vh16[e] = __builtin_bit_cast(_Float16,
                                                     *reinterpret_cast<const uint16_t*>(vtile + (8 * g + e) * ROW + c * 2));
                    else
                        vh16[e] = static_cast<_Float16>(elem_f32<FMT>(vtile + (8 * g + e) * ROW + c * ES));
                }
                acc[nd] = mfma_h(vh16, ph16, acc[nd]);
                acc[nd] = mfma_h(vh16, pl16, acc[nd]);
                continue;
            }
            bf16x8 vh, vl;
            if constexpr (FMT == BF16) {  // the staged bits are the operand (no widening and rounding back)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    vh[e] = __builtin_bit_cast(__bf16, *reinterpret_cast<const uint16_t*>(vtile + (8 * g + e) * ROW + c * 2));
            } else {
                float x[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = elem_f32<FMT>(vtile + (8 * g + e) * ROW + c * ES);
                split8(x, vh, vl);
            }
            acc[nd] = mfma(vh, ph, acc[nd]);
            acc[nd] = mfma(vh, pl, acc[nd]);
            if constexpr (KLO) acc[nd] = mfma(vl, ph, acc[nd]);
        }
    };

    // KP: the wave's leading tiles of codes only (keys and values quantized, the tile's keys inside one key group,
    // value groups that hold whole chunks) are pipelined like the register buffers of the dense path: the next
    // tile's codes, scales and zero points (a few registers per chunk) are loaded while a tile is dequantized into
    // LDS and computed; every later tile is staged as it comes.
    constexpr bool KP_PIPE = KP && DP <= 128 && !MASKED;
    // (TWO: a tile may span two key groups, groups of 16 or 24 tokens; else every tile lies in one)
    auto codes_run = [&](auto bits_c, auto two_c, int n) __attribute__((always_inline)) {
        constexpr int BITS = decltype(bits_c)::value;
        constexpr bool TWO = decltype(two_c)::value;
        constexpr int NB = CE * BITS / 8;
        constexpr int NW = NB > 4 ? 2 : 1;  // code words of a chunk
        struct CodesRaw {
            uint32_t kc[KP_PIPE ? KCH : 1][NW], vc[KP_PIPE ? VCH : 1][NW];
            uint4 ks[TWO ? 2 : 1], kz[TWO ? 2 : 1];  // the scales and zero points of the tile's key groups
            uint16_t vs[KP_PIPE ? VCH : 1], vz[KP_PIPE ? VCH : 1];
            int split_at;  // the tile's first token of its last key group
        };
        auto words = [](uint2 w, uint32_t (&out)[NW]) __attribute__((always_inline)) {
            out[0] = w.x;
            if constexpr (NW == 2) out[NW - 1] = w.y;
        };
        auto pair = [](const uint32_t (&in)[NW]) __attribute__((always_inline)) {
            return make_uint2(in[0], NW == 2 ? in[NW - 1] : 0u);
        };
        const int kc0 = (lane % KCR) * CE, vc0 = v0 + (lane % VCR) * CE;
        const bool k_ok = kc0 < p.head_dim, v_ok = vc0 < p.value_dim;
        const int kcc = k_ok ? kc0 : 0, vcc = v_ok ? vc0 : 0;
        auto load = [&](CodesRaw& R, Keys& K, int k) __attribute__((always_inline)) {
            issue(K, k);  // (the mask bytes)
            const int t0 = tile_start(k);
#pragma unroll
            for (int i = 0; i < KCH; ++i) {
                const int t = t0 + (lane + 64 * i) / KCR;
                words(load_code_bytes<NB>(kcb + static_cast<int64_t>(t) * p.skc_s + kcc * BITS / 8), R.kc[i]);
            }
            const int g0 = t0 / p.kp_kg, g1 = (t0 + TK - 1) / p.kp_kg;  // g1 <= g0 + 1 on this path
            R.split_at = g1 * p.kp_kg;
#pragma unroll
            for (int j = 0; j < (TWO ? 2 : 1); ++j) {
                const int64_t so = static_cast<int64_t>(j ? g1 : g0) * p.sks_g + kcc;
                R.ks[j] = load_halves<CE>(ksb + so);
                R.kz[j] = load_halves<CE>(kzb + so);
            }
#pragma unroll
            for (int i = 0; i < VCH; ++i) {
                const int t = t0 + (lane + 64 * i) / VCR;
                words(load_code_bytes<NB>(vcb + static_cast<int64_t>(t) * p.svc_s + vcc * BITS / 8), R.vc[i]);
                const int64_t vo = static_cast<int64_t>(t) * p.svs_s + vcc / p.kp_vg;
                R.vs[i] = vsb[vo];
                R.vz[i] = vzb[vo];
            }
        };
        auto fill = [&](const CodesRaw& R, int t0) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < KCH; ++i) {
                const bool last = TWO && t0 + (lane + 64 * i) / KCR >= R.split_at;
                const f16x8 s8 = __builtin_bit_cast(f16x8, last ? R.ks[TWO ? 1 : 0] : R.ks[0]);
                const f16x8 z8 = __builtin_bit_cast(f16x8, last ? R.kz[TWO ? 1 : 0] : R.kz[0]);
                float c[8], x[CE];
                chunk_codes<BITS>(pair(R.kc[i]), c);
#pragma unroll
                for (int e = 0; e < CE; ++e)
                    x[e] = __builtin_fmaf(c[e], static_cast<float>(s8[e]), static_cast<float>(z8[e]));
                *reinterpret_cast<uint4*>(ktile + ((lane + 64 * i) / KCR) * KROW + kc0 * ES) =
                    k_ok ? pack_chunk<FMT>(x) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < VCH; ++i) {
                const float sc = half_f32(R.vs[i]), zr = half_f32(R.vz[i]);
                float c[8], x[CE];
                chunk_codes<BITS>(pair(R.vc[i]), c);
#pragma unroll
                for (int e = 0; e < CE; ++e) x[e] = __builtin_fmaf(c[e], sc, zr);
                *reinterpret_cast<uint4*>(vtile + ((lane + 64 * i) / VCR) * ROW + (vc0 - v0) * ES) =
                    v_ok ? pack_chunk<FMT>(x) : make_uint4(0, 0, 0, 0);
            }
        };
        // past the run's last tile every step loads that tile again (read from L2 and never used)
        CodesRaw RA, RB;
        Keys KA, KB;
        int ki = 0, k = 0;
        load(RA, KA, 0);
        while (true) {
            ki = min(ki + 1, n - 1);
            load(RB, KB, ki);
            fill(RA, tile_start(k));
            compute(KA, tile_start(k));
            if (++k >= n) break;
            ki = min(ki + 1, n - 1);
            load(RA, KA, ki);
            fill(RB, tile_start(k));
            compute(KB, tile_start(k));
            if (++k >= n) break;
        }
    };

    if (my_tiles > 0) {
        if constexpr (KP) {
            int k = 0;
            if constexpr (KP_PIPE) {
                // tiles split + k splits lying wholly below both quantized counts, a prefix of the wave's tiles, when
                // no tile spans more than two key groups (groups of at least 32 tokens, or of 16 or 24, whose
                // boundaries fall at most once inside an aligned 32-token tile) and value groups hold whole chunks
                const int below = min(kq, vq) / TK;
                int n = split < below ? (below - 1 - split) / p.splits + 1 : 0;
                const int kg = p.kp_kg;
                if (!(kg >= TK || kg == 16 || kg == 24) || p.kp_vg % CE != 0) n = 0;
                n = min(n, my_tiles);
                const bool two = kg % TK != 0;
                if (two && p.kp_bits == 8) n = 0;  // (two buffers of 8-bit codes and two key groups: too many registers)
                if (n > 0) {
                    using I2 = std::integral_constant<int, 2>;
                    using I4 = std::integral_constant<int, 4>;
                    using I8 = std::integral_constant<int, 8>;
                    if (two) {
                        if (p.kp_bits == 2)
                            codes_run(I2{}, std::true_type{}, n);
                        else
                            codes_run(I4{}, std::true_type{}, n);
                    } else if (p.kp_bits == 2) {
                        codes_run(I2{}, std::false_type{}, n);
                    } else if (p.kp_bits == 4) {
                        codes_run(I4{}, std::false_type{}, n);
                    } else {
                        codes_run(I8{}, std::false_type{}, n);
                    }
                }
                k = n;
            }
            for (; k < my_tiles; ++k) {
                Keys K;
                issue(K, k);
                stage(tile_start(k));
                compute(K, tile_start(k));
            }
        } else if constexpr (NBUF == 1) {
            for (int k = 0; k < my_tiles; ++k) {
                Keys K;
                issue(K, k);
                stage(tile_start(k));
                compute(K, tile_start(k));
            }
        } else {
            // past the wave's last tile every step issues that tile again (read from L2 and never computed)
            Keys K0, K1;
            int ki = 0, k = 0;
            issue(K0, ki);
            while (true) {
                stage(tile_start(k));
                ki = min(ki + 1, my_tiles - 1);
                issue(K1, ki);
                compute(K0, tile_start(k));
                if (++k >= my_tiles) break;
                stage(tile_start(k));
                ki = min(ki + 1, my_tiles - 1);
                issue(K0, ki);
                compute(K1, tile_start(k));
                if (++k >= my_tiles) break;
            }
        }
    }
    l_i = group_sum(l_i);
    const float sink = p.sinks && r_ok ? p.sinks[h] * kLog2e : -INFINITY;
    auto out_at = [&](int row_qi, int row_h, int d) __attribute__((always_inline)) -> int64_t {
        return b * p.so_b + static_cast<int64_t>(q_start + row_qi) * p.so_q + row_h * p.so_h + d;
    };

    // ---- one split: the row's output directly; lane (n, g) holds channels 16 nd + 4 g + i of row r ----
    if (p.splits == 1) {
        if (!r_ok) return;
        float inv;
        const float a = sink_weight(m_i, l_i, sink, inv);
#pragma unroll
        for (int nd = 0; nd < ND; ++nd)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = v0 + 16 * nd + 4 * g + i;
                if (d < p.value_dim) store_out<QF>(p, out_at(qi, h, d), acc[nd][i] * vs * a * inv);
            }
        return;
    }

    // ---- the split's partial: row n's max and sum (lane group 0) and its channels 16 nd + 4 g + i ----
    const int64_t slot_stride = DP + 2;
    const int64_t prog_part = static_cast<int64_t>(prog) * p.splits * 16;
    if (r_ok) {
        float* slot = p.part + (prog_part + split * 16 + n) * slot_stride;
        if (g == 0 && blockIdx.z == 0) {  // (every value slice has the same maximum and sum)
            coherent_store(slot, m_i);
            coherent_store(slot + 1, l_i);
        }
#pragma unroll
        for (int nd = 0; nd < ND; ++nd)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (v0 + 16 * nd < p.value_dim) coherent_store(slot + 2 + v0 + 16 * nd + 4 * g + i, acc[nd][i] * vs);
    }
    // The hand-off to the last split to finish: the partials are written and read as agent-scope atomics (sc1), so
    // completion orders them; the compiler may not move the stores past the count (a signal fence), the wave waits
    // for its stores (vmcnt counts stores on gfx950), then lane 0 counts the split; the wave that finds every other
    // split counted loads the partials after its atomic returned and leaves the counter zero for the next call.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    int prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(p.counters + prog, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__shfl(prev, 0) != p.splits * static_cast<int>(gridDim.z) - 1) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);

    // ---- the merge by log-sum-exp: lane-owned runs of 8 channels of one query row, the splits folded in batches of 4
    // with their loads in flight together ----
    const int rows_here = min(16, p.rows - mt * 16);
    for (int base = 0; base < rows_here * p.value_dim; base += 64 * 8) {
        const int e = base + lane * 8;
        const bool active = e < rows_here * p.value_dim;
        const int rr = active ? e / p.value_dim : 0;
        const int d = active ? e % p.value_dim : 0;
        const int row = mt * 16 + rr;
        const int row_qi = row % p.queries, row_h = kvh * p.groups + row / p.queries;
        const bool live = active && row_qi < q_count;
        float m_run = -INFINITY, l_run = 0.0f, o_run[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o_run[i] = 0.0f;
        for (int s0 = 0; s0 < p.splits; s0 += 4) {
            float mk[4], lk[4], ok[4][8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool use = live && s0 + j < p.splits;
                const float* sk = p.part + (prog_part + (use ? s0 + j : 0) * 16 + rr) * slot_stride;
                mk[j] = use ? coherent_load(sk) : -INFINITY;
                lk[j] = use ? coherent_load(sk + 1) : 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) ok[j][i] = use ? coherent_load(sk + 2 + d + i) : 0.0f;
            }
            float m_new = m_run;
#pragma unroll
            for (int j = 0; j < 4; ++j) m_new = fmaxf(m_new, mk[j]);
            if (m_new == -INFINITY) continue;
            const float a = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= a;
#pragma unroll
            for (int i = 0; i < 8; ++i) o_run[i] *= a;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (mk[j] == -INFINITY) continue;
                const float cw = __builtin_amdgcn_exp2f(mk[j] - m_new);
                l_run += lk[j] * cw;
#pragma unroll
                for (int i = 0; i < 8; ++i) o_run[i] += ok[j][i] * cw;
            }
            m_run = m_new;
        }
        if (live) {
            const float row_sink = p.sinks ? p.sinks[row_h] * kLog2e : -INFINITY;
            float inv;
            const float a = sink_weight(m_run, l_run, row_sink, inv);
#pragma unroll
            for (int i = 0; i < 8; ++i) store_out<QF>(p, out_at(row_qi, row_h, d + i), o_run[i] * a * inv);
        }
    }
    if (lane == 0) __hip_atomic_store(p.counters + prog, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

}  // namespace eco
