// KIVI (Liu et al., ICML 2024) on gfx950: the quantization schedule, the full-precision residual ring,
// quantize-and-append into 32-token pages, and decode attention that feeds the codes to the matrix cores.
//
// Quantization follows the reference's quantize (techniques/kv_quant/kivi.py:121-140): fp32 min and max along the
// group; scale = fp16r((high - low) / levels) and low = fp16r(low), fp16r rounding to nearest even where fp16 holds
// the value; codes = round_half_even((x - low) / safe) clamped to [0, levels], safe = scale or 1 where the scale is 0.
// Both divisions are IEEE divisions (__fdiv_rn), the CPU semantics of torch's tensor / int and tensor / tensor (GPU
// torch multiplies by a reciprocal instead; the parity oracle is the CPU definition). Keys are quantized per channel
// over a 32-token group (one page), values per token over 32-channel groups. The schedule is the reference's
// (kivi.py:230-243): with c committed tokens, keys below (c / R) * R and values below max(0, c - R) are quantized.
//
// Page block (one per (page, KV head), offsets in KiviLayout): key codes token-major, each token's channels packed
// in 32-bit words; value codes as words (u * 16 + n) * (D / 16) + nd, channel 16 nd + n, tokens u * 32 / bits ..;
// key scales and zero points [D]; value scales and zero points [D / 32][32]. A word holds 32 / bits elements,
// element e in byte e % 4 at bit (e / 4) * bits.
//
// Attention. The reference dequantizes code * scale + zero in fp32 and attends over the keys and values rounded to
// the model dtype (attention/kivi.py:56-76, attention/_kivi_kernels.py:14-15 and the .to(DOT_DTYPE) casts of
// _kivi_block). Both are dequantized that way here: a code c < 16 zero-extended to a byte is the e4m3 pattern of
// c * 2^-9, so v_cvt_scalef32_pk_f32_fp8 with scale 2^9 gives the exact fp32 value c; c * s is exact in fp32 (at
// most 4 bits times an fp16), so one fused multiply-add rounds as the reference's product then sum; the result is
// rounded to bf16 and fed to bf16 MFMAs. The value product's B operand p is split into two bf16 terms (hi + lo,
// about 16 significant bits), so the output carries the reference's value rounding and nothing coarser; every
// product is in fp32 (no fp16 operand, whatever the scale). Tokens not yet quantized are read from the bf16 ring.
//
// Work decomposition, pipeline and merge: the stream-K scheme of paged_attention.hip (stream_k.hpp), with tiles of
// one 32-token page. The query of the current row lives in LDS, so that row changes do not put loads of varying
// count in the tile pipeline. More than 32 query rows per KV head (speculative verification) go to kivi_verify.hip.

#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "kivi.hpp"
#include "kivi_math.hpp"
#include "stream_k.hpp"

namespace eco {

namespace {

constexpr int KPAGE = KiviParams::kPage;  // 32 tokens

__device__ inline float load_elem(const void* base, int64_t offset, int format) {
    if (format == BF16) return bf16_to_f32(static_cast<const uint16_t*>(base)[offset]);
    if (format == FP16) return static_cast<float>(static_cast<const _Float16*>(base)[offset]);
    return static_cast<const float*>(base)[offset];
}

__device__ inline uint16_t f16_bits(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// ---- schedule --------------------------------------------------------------------------------------------------

// ranges [4][B]: keys [from, to), values [from, to) to quantize now; the counts advance to their new values.
__global__ void kivi_schedule_kernel(const int32_t* committed, int residual, int32_t* kq, int32_t* vq,
                                     int32_t* ranges, int batch) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= batch) return;
    const int c = max(committed[b], 0);
    const int k_to = max(kq[b], (c / residual) * residual);
    const int v_to = max(vq[b], c - residual);
    ranges[b] = kq[b];
    ranges[batch + b] = k_to;
    ranges[2 * batch + b] = vq[b];
    ranges[3 * batch + b] = v_to;
    kq[b] = k_to;
    vq[b] = v_to;
}

// ---- residual ring ------------------------------------------------------------------------------------------

// One workgroup per new token: keys to slot t % W of [B, Hkv, W, D], values to [B, Hkv, D, W], rounded to bf16.
__global__ __launch_bounds__(256) void kivi_ring_kernel(KiviRingParams p) {
    const int t = blockIdx.x;
    const int pos = p.positions[t];
    const int b = p.rows[t];
    if (pos < 0 || b < 0 || b >= p.batch) return;
    const int slot = pos % p.ring;
    for (int i = threadIdx.x; i < p.kv_heads * p.head_dim; i += blockDim.x) {
        const int h = i / p.head_dim, d = i % p.head_dim;
        const float k = load_elem(p.k_new, t * p.sk_t + h * p.sk_h + d, p.in_format);
        const float v = load_elem(p.v_new, t * p.sv_t + h * p.sv_h + d, p.in_format);
        const int64_t row = static_cast<int64_t>(b) * p.kv_heads + h;
        p.k_ring[(row * p.ring + slot) * p.head_dim + d] = f32_to_bf16(k);
        p.v_ring[(row * p.head_dim + d) * p.ring + slot] = f32_to_bf16(v);
    }
}

// ---- quantize-and-append ----------------------------------------------------------------------------------------

__device__ inline float src_elem(const KiviQuantParams& p, int b, int h, int t, int d) {
    const int slot = p.src_ring > 0 ? t % p.src_ring : t - p.src_start;
    return load_elem(p.src, b * p.ss_b + h * p.ss_h + static_cast<int64_t>(slot) * p.ss_t + d * p.ss_d,
                     p.src_format);
}

__device__ inline uint8_t* page_block(const KiviQuantParams& p, int b, int h, int page) {
    if (page >= p.bt_cols) return nullptr;
    const int phys = p.block_table[b * p.bt_stride + page];
    if (phys < 0 || phys >= p.num_pages) return nullptr;
    return p.blocks + static_cast<int64_t>(phys) * p.blk_page + h * p.blk_head;
}

// Keys: one workgroup per (row, KV head) and 32-token group in [from, to) (multiples of 32).
__global__ __launch_bounds__(256) void kivi_quant_keys_kernel(KiviQuantParams p) {
    __shared__ float s_low[256], s_safe[256];
    const int row = blockIdx.x;
    const int b = row / p.kv_heads, h = row % p.kv_heads;
    const int page = p.from[b] / KPAGE + static_cast<int>(blockIdx.y);
    const int t0 = page * KPAGE;
    if (t0 + KPAGE > p.to[b]) return;
    uint8_t* blk = page_block(p, b, h, page);
    if (!blk) return;
    const KiviLayout L{p.head_dim, p.bits};
    const int levels = (1 << p.bits) - 1;
    for (int d = threadIdx.x; d < p.head_dim; d += blockDim.x) {
        float lo = INFINITY, hi = -INFINITY;
        for (int t = 0; t < KPAGE; ++t) {
            const float x = src_elem(p, b, h, t0 + t, d);
            lo = fminf(lo, x);
            hi = fmaxf(hi, x);
        }
        const Quant q = make_quant(lo, hi, levels, p.overflow);
        s_low[d] = q.low;
        s_safe[d] = q.safe;
        reinterpret_cast<uint16_t*>(blk + L.k_scale())[d] = f16_bits(q.scale);
        reinterpret_cast<uint16_t*>(blk + L.k_zero())[d] = f16_bits(q.low);
    }
    __syncthreads();
    const int per_word = 32 / p.bits;
    const int words = p.head_dim / per_word;  // per token
    for (int item = threadIdx.x; item < KPAGE * words; item += blockDim.x) {
        const int t = item / words, w = item % words;
        uint32_t word = 0;
        for (int e = 0; e < per_word; ++e) {
            const int d = w * per_word + e;
            const Quant q{0.0f, s_low[d], s_safe[d]};
            word |= code_of(src_elem(p, b, h, t0 + t, d), q, levels) << (8 * (e & 3) + (e >> 2) * p.bits);
        }
        reinterpret_cast<uint32_t*>(blk + L.k_codes() + t * (p.head_dim * p.bits / 8))[w] = word;
    }
}

// Values: one workgroup per (row, KV head) and page overlapping [from, to); the page's other tokens keep their codes.
__global__ __launch_bounds__(256) void kivi_quant_values_kernel(KiviQuantParams p) {
    __shared__ float s_low[KPAGE][8], s_safe[KPAGE][8];
    const int row = blockIdx.x;
    const int b = row / p.kv_heads, h = row % p.kv_heads;
    const int page = p.from[b] / KPAGE + static_cast<int>(blockIdx.y);
    const int t0 = page * KPAGE;
    const int lo_t = max(p.from[b], t0), hi_t = min(p.to[b], t0 + KPAGE);
    if (lo_t >= hi_t) return;
    uint8_t* blk = page_block(p, b, h, page);
    if (!blk) return;
    const KiviLayout L{p.head_dim, p.bits};
    const int levels = (1 << p.bits) - 1;
    const int groups = p.head_dim / 32;
    for (int item = threadIdx.x; item < (hi_t - lo_t) * groups; item += blockDim.x) {
        const int t = lo_t + item / groups, grp = item % groups;
        float lo = INFINITY, hi = -INFINITY;
        for (int d = 32 * grp; d < 32 * grp + 32; ++d) {
            const float x = src_elem(p, b, h, t, d);
            lo = fminf(lo, x);
            hi = fmaxf(hi, x);
        }
        const Quant q = make_quant(lo, hi, levels, p.overflow);
        s_low[t - t0][grp] = q.low;
        s_safe[t - t0][grp] = q.safe;
        reinterpret_cast<uint16_t*>(blk + L.v_scale())[grp * KPAGE + (t - t0)] = f16_bits(q.scale);
        reinterpret_cast<uint16_t*>(blk + L.v_zero())[grp * KPAGE + (t - t0)] = f16_bits(q.low);
    }
    __syncthreads();
    const int per_word = 32 / p.bits;  // tokens per word
    const int nd_count = p.head_dim / 16;
    uint32_t* words = reinterpret_cast<uint32_t*>(blk + L.v_codes());
    for (int item = threadIdx.x; item < p.bits * 16 * nd_count; item += blockDim.x) {
        const int u = item / (16 * nd_count);
        const int n = (item / nd_count) % 16;
        const int nd = item % nd_count;
        const int d = 16 * nd + n;
        const int w0 = t0 + u * per_word;  // first token of the word
        if (w0 + per_word <= lo_t || w0 >= hi_t) continue;
        uint32_t word = words[item];
        for (int e = 0; e < per_word; ++e) {
            const int t = w0 + e;
            if (t < lo_t || t >= hi_t) continue;
            const int shift = 8 * (e & 3) + (e >> 2) * p.bits;
            const Quant q{0.0f, s_low[t - t0][d / 32], s_safe[t - t0][d / 32]};
            word = (word & ~(static_cast<uint32_t>(levels) << shift)) | (code_of(src_elem(p, b, h, t, d), q, levels) << shift);
        }
        words[item] = word;
    }
}

// ---- attention ----------------------------------------------------------------------------------------------

// A lane's share of one 32-token page: key words of its 8-token key rows, the value word of each 16-channel block
// (lane (n, g): channel 16 nd + n, tokens 8 g .. 8 g + 7, the P.V MFMA's A operand) and D / 8 bytes of the page's
// scales and zero points (8 D contiguous bytes of the page block: key scales, key zero points, value scales, value
// zero points; lane l holds bytes l D / 8 ..). The 16 lanes of a lane group use the same scales, so the tile's compute
// writes the 64 lanes' shares to an LDS slot of the wave and each lane reads what it uses from there: four registers
// per tile buffer instead of sixty-four.
template <int D, int BITS>
struct KTile {
    static constexpr int KW = D * BITS / 128;  // words of a lane's key slice (D / 4 channels)
    static constexpr int ND = D / 16;          // value blocks of 16 channels
    static constexpr int KS = D / 32;          // k-steps of an S MFMA (8 channels each per lane)
    static constexpr int VG = D / 32;          // value groups
    static constexpr int SCALE_BYTES = 8 * D;  // the page's scales and zero points
    using Share = typename std::conditional<D == 128, uint4, uint2>::type;  // a lane's D / 8 bytes of them
    static_assert(sizeof(Share) * 64 == SCALE_BYTES, "64 lanes hold the scales");
    uint32_t kc[2][KW];
    uint32_t vc[ND];
    Share sc;
    int page;          // physical page (the same in every lane), -1 for none
    uint32_t mw[4];    // with a mask: bit e = token 8 g + e of the page visible to query row 16 nb + n (nb < NB)
};

// N code words from src, streamed (codes are read once per call; C3 at L=8192, int2 / int4: 55.7 / 57.6 us plain,
// 52.6 / 55.1 us streamed).
template <int N>
__device__ inline void load_words(const uint32_t* src, uint32_t (&dst)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const uint4 w = stream_load16(src + i);
            dst[i] = w.x;
            dst[i + 1] = w.y;
            dst[i + 2] = w.z;
            dst[i + 3] = w.w;
        }
    } else if constexpr (N == 2) {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(src));
        const uint2 w = make_uint2(x.x, x.y);
        dst[0] = w.x;
        dst[1] = w.y;
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

// A row's tiles are walked from its last one down (at_tile: position t of the cursor is tile tiles - 1 - t). The
// row's newest tokens, its bf16 ring tiles (not yet quantized; their loads are issued inside the tile step and
// waited for at once), then come first, while every wave's pipeline is filling anyway, instead of in the last part
// of the row, whose workgroup would then also finish last and run the row's merge.

// Issues the page loads of tile c.t of c's row (the same loads in every lane and for every tile: a tile without a
// page reads page 0 and masks it).
template <int D, int BITS>
__device__ __forceinline__ void issue_tile(const KiviParams& p, const Cursor& c, int n, int g, int lane, PageWindow& win,
                                           KTile<D, BITS>& tile) {
    using T = KTile<D, BITS>;
    constexpr KiviLayout L{D, BITS};
    ensure_window<KiviParams, true>(p, c, lane, win);
    const int phys = __builtin_amdgcn_readlane(win.physical, c.t - win.base);
    tile.page = phys;
    const uint8_t* blk = p.blocks + static_cast<int64_t>(phys >= 0 ? phys : 0) * p.blk_page + c.kvh * p.blk_head;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
        const int token = 8 * (n >> 2) + 4 * v + (n & 3);
        load_words(reinterpret_cast<const uint32_t*>(blk + L.k_codes() + token * (D * BITS / 8)) + g * T::KW, tile.kc[v]);
    }
    constexpr int TPW = 32 / BITS;  // tokens per value word
    const int u = 8 * g / TPW;
    load_words(reinterpret_cast<const uint32_t*>(blk + L.v_codes()) + (u * 16 + n) * T::ND, tile.vc);
    static_assert(L.k_zero() == L.k_scale() + 2 * D && L.v_zero() == L.k_scale() + 6 * D, "scales contiguous");
    tile.sc = *reinterpret_cast<const typename T::Share*>(blk + L.k_scale() + lane * sizeof(typename T::Share));
}

// The eight values (tokens 8 g .. 8 g + 7 of one channel) of a value word, dequantized as the reference does:
// bf16(code * scale + zero) with the product and sum in fp32 (one fused multiply-add: the product is exact).
template <int BITS>
__device__ __forceinline__ uint4 dequant_values(uint32_t word, int g, const uint4& scales, const uint4& zeros) {
    const f16x8 sh = __builtin_bit_cast(f16x8, scales);
    const f16x8 zh = __builtin_bit_cast(f16x8, zeros);
    float c8[8];
    codes_to_f32<BITS>(word, BITS == 4 ? 0 : (g & 1), c8);
    bf16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        v[i] = static_cast<__bf16>(__builtin_fmaf(c8[i], static_cast<float>(sh[i]), static_cast<float>(zh[i])));
    return __builtin_bit_cast(uint4, v);
}

// Masks of the bf16 halves of a uint4 whose bit in keep (8 bits, element e = bit e) is set.
struct HalfMask {
    uint32_t m[4];
};

__device__ inline HalfMask half_mask(uint32_t keep) {
    HalfMask h;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        h.m[j] = ((keep >> (2 * j)) & 1u ? 0x0000FFFFu : 0u) | ((keep >> (2 * j + 1)) & 1u ? 0xFFFF0000u : 0u);
    return h;
}

__device__ inline uint4 apply_mask(uint4 x, const HalfMask& h) {
    return make_uint4(x.x & h.m[0], x.y & h.m[1], x.z & h.m[2], x.w & h.m[3]);
}

// p (8 fp32 weights) as bf16 hi + lo: hi = bf16(p), lo = bf16(p - hi) (p - hi is exact in fp32).
__device__ __forceinline__ void split_bf16(const float (&p)[8], bf16x8& hi, bf16x8& lo) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        hi[e] = static_cast<__bf16>(p[e]);
        lo[e] = static_cast<__bf16>(p[e] - static_cast<float>(hi[e]));
    }
}

}  // namespace

// Workgroup shapes. One column block at D <= 128: four waves split the workgroup's tile range in quarters, the
// pieces of rows inside the workgroup merged through LDS (as in paged_attention.hip). Otherwise one wave.
template <int D, int NB>
constexpr int kivi_wg_waves() {
    return NB == 1 && D <= 128 ? 4 : 1;
}

// Waves per SIMD of the one-column-block instances: two with two tile buffers; with one, three where the pieces hold
// at most 8 query rows and the registers fit (D = 64), else two. One wave of a SIMD does not overlap its own
// arithmetic with its outstanding loads, more waves do.
template <int D, int NB, int NBUF, int PR>
constexpr int kivi_waves_per_simd() {
    return NB == 1 && D <= 128 ? (NBUF == 1 && PR <= 8 && D == 64 ? 3 : 2) : 1;
}

// PR: the query rows a piece of the split instances holds (4, 8 or 16; at least the shape's rows): the LDS of a
// workgroup, and with it the workgroups a CU holds, follows the rows a shape has instead of the MFMA's 16 columns.
template <int D, int BITS, int NB, int NBUF, int PR>
__global__ __launch_bounds__((64 * kivi_wg_waves<D, NB>()))
    __attribute__((amdgpu_waves_per_eu(kivi_waves_per_simd<D, NB, NBUF, PR>()))) void
kivi_attention_kernel(KiviParams p) {
    using T = KTile<D, BITS>;
    constexpr int KS = T::KS, ND = T::ND, VG = T::VG;
    constexpr int R = NB * 16;  // query rows of the MFMA columns
    constexpr int WAVES = kivi_wg_waves<D, NB>();
    constexpr bool kSplit = WAVES > 1;  // the range split in quarters, pieces merged in LDS
    static_assert(PR == 16 || (kSplit && NB == 1), "pieces of fewer rows only for the split instances");
    // a wave's current query rows (one word of padding: a row stride of D / 8 + 1 words puts the 16 rows of a lane
    // group in distinct banks); with pieces of PR < 16 rows, the PR rows and a zero row read by MFMA columns PR .. 15
    constexpr int QR = PR < 16 ? PR + 1 : R;
    using QRows = uint4[QR][D / 8 + 1];

    const int lane = WAVES > 1 ? static_cast<int>(threadIdx.x) & 63 : static_cast<int>(threadIdx.x);
    const int wave = WAVES > 1 ? uniform(static_cast<int>(threadIdx.x) >> 6) : 0;
    constexpr int row0 = 0;  // the first query row of the wave's columns
    __shared__ __align__(16) typename std::conditional<kSplit, Pieces<D, WAVES, PR>, char>::type pieces;
    // the scales and zero points of the tile a wave computes
    __shared__ __align__(16) uint8_t scale_slots[WAVES][T::SCALE_BYTES];
    QRows* q_rows;
    if constexpr (kSplit) {
        // the query rows live in the data of the wave's second piece, which only the wave's last step writes, after
        // its last read of them (the piece's row, b, kvh and tiles fields lie outside the data)
        static_assert(sizeof(QRows) <= sizeof(pieces.data[0]), "query rows fit a piece");
        q_rows = reinterpret_cast<QRows*>(pieces.data[2 * wave + 1]);
    } else {
        __shared__ QRows q_lds[WAVES];
        q_rows = &q_lds[wave];
    }
    auto& q_bf = *q_rows;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int qn = PR < 16 ? min(n, PR) : n;  // the query row of MFMA column n
    const int w = xcd_range(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));  // the workgroup's range
    const int grid = gridDim.x;

    // row geometry: one load of the lengths for batches of at most 64 rows
    const bool small = p.batch <= 64;
    RowTable rt{};
    if (small) rt = row_table(p, lane);
    const int64_t total = small ? uniform64(__shfl(rt.incl, 63)) : uniform64(total_tiles(p, lane));
    for (int b = w * WAVES + wave; b < p.batch; b += grid * WAVES) {  // rows without a key: zeros
        if ((small ? __builtin_amdgcn_readlane(rt.row.tiles, b) : row_of(p, b).tiles) == 0)
            for (int idx = lane; idx < p.kv_heads * p.rows * D; idx += 64)
                store_output(p, b, idx / (p.rows * D), (idx / D) % p.rows, idx % D, 0.0f, -INFINITY, 0.0f);
    }
    const int64_t wlo = total * w / grid;  // the workgroup's tile range
    const int64_t whi = total * (w + 1) / grid;
    const int64_t lo = kSplit ? wlo + (whi - wlo) * wave / WAVES : wlo;  // this wave's part of it
    const int64_t hi = kSplit ? wlo + (whi - wlo) * (wave + 1) / WAVES : whi;
    if constexpr (kSplit) {
        clear_pieces(pieces, wave, lane);
    } else {
        if (lo >= hi) return;
    }

    // ---- row state ----
    float limit[NB];
    int all_see = 0, kq = 0, vq = 0, row_len = 0;
    float m_i[NB], l_i[NB];  // l_i: the sum over the lane's own tokens until the segment's end reduces it
    f32x4 acc[ND][NB];

    auto begin_row = [&](const Cursor& c) __attribute__((always_inline)) {
        // the row's query rows into LDS (rows past the group are zero); the loads wait here, once per row, outside the
        // tile pipeline
        for (int i = lane; i < QR * (D / 8); i += 64) {
            const int r = i / (D / 8), k = i % (D / 8);
            uint4 x = make_uint4(0, 0, 0, 0);
            if (row0 + r < p.rows) {
                const int gq = (row0 + r) / p.queries, qi = (row0 + r) % p.queries;
                x = *reinterpret_cast<const uint4*>(p.q + c.b * p.sq_b + qi * p.sq_q +
                                                    (c.kvh * p.groups + gq) * p.sq_h + 8 * k);
            }
            q_bf[r][k] = x;
        }
        __builtin_amdgcn_s_waitcnt(0);
        kq = scalar_load(p.keys_quantized, c.b);
        vq = scalar_load(p.values_quantized, c.b);
        row_len = c.row.len;
        all_see = c.row.len - p.queries - p.queries_after + 1;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int r = row0 + nb * 16 + n;
            limit[nb] = r < p.rows ? static_cast<float>(c.row.len - p.queries - p.queries_after + r % p.queries + 1) : 0.0f;
            // the accumulators are cleared by the row's first rescale (m_i = -inf marks a row with no weight yet),
            // so that a row change does not give them a second register version to merge at every tile
            m_i[nb] = -INFINITY;
            l_i[nb] = 0.0f;
        }
    };
    const float score_scale = p.softcap > 0.0f ? p.scale : p.scale * kLog2e;

    // the value tokens 8 g .. 8 g + 7 of the lane that come from codes (below vq, on a present page)
    auto code_values = [&](const T& tile, int t0) __attribute__((always_inline)) -> uint32_t {
        const int tok0 = t0 + 8 * g;
        if (tile.page < 0) return 0u;
        return vq - tok0 >= 8 ? 0xFFu : (vq > tok0 ? (1u << (vq - tok0)) - 1u : 0u);
    };

    // ---- one tile (32 tokens) of the online softmax ----
    auto compute = [&](const T& tile, const Cursor& c) __attribute__((always_inline)) {
        // the tile's scales into the wave's slot (the previous tile's reads of it came first: one wave's LDS accesses
        // are in order)
        uint8_t* sl = scale_slots[wave];
        reinterpret_cast<typename T::Share*>(sl)[lane] = tile.sc;
        const int t0 = KPAGE * at_tile(c).t;
        const bool valid = tile.page >= 0;
        f32x4 s[2][NB];
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s[v][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // the lane's value word of each 16-channel block from the ring (tokens 8 g .. 8 g + 7 of the tile, channel
        // 16 nd + n): read with the ring keys when both halves of the tile hold ring tokens, so that such a tile waits
        // out one load round trip instead of two (up to two column blocks: at four the registers would spill)
        constexpr bool kJointRing = NB <= 2;
        const int tok0 = t0 + 8 * g;
        const bool key_ring = t0 >= kq, value_ring = t0 + KPAGE > vq;
        uint4 vr[ND];
        auto load_value_ring = [&]() __attribute__((always_inline)) {
            const int slot = tok0 % p.ring;
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
                vr[nd] = *reinterpret_cast<const uint4*>(
                    p.v_ring + ((static_cast<int64_t>(c.b) * p.kv_heads + c.kvh) * D + 16 * nd + n) * p.ring + slot);
        };
        // keys from codes, dequantized as the reference does (code * scale + zero in fp32, two roundings, then bf16;
        // attention/kivi.py:56-76), so that the scores see the reference's key values exactly; or, at or past kq,
        // from the ring (kq counts whole 32-token key groups, so a page is either all codes or all ring)
        if (!key_ring) {
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const f16x8 sh = *reinterpret_cast<const f16x8*>(sl + (g * (D / 4) + 8 * j) * 2);
                const f16x8 zh = *reinterpret_cast<const f16x8*>(sl + 2 * D + (g * (D / 4) + 8 * j) * 2);
                float sf[8], zf[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    sf[e] = static_cast<float>(sh[e]);
                    zf[e] = static_cast<float>(zh[e]);
                }
#pragma unroll
                for (int v = 0; v < 2; ++v) {
                    float c8[8];
                    codes_to_f32<BITS>(BITS == 4 ? tile.kc[v][j] : tile.kc[v][j / 2], j % 2, c8);
                    bf16x8 kv;
                    // code * scale is exact in fp32 (a code of at most 4 bits times an fp16), so one fused
                    // multiply-add rounds exactly as the reference's product then sum
#pragma unroll
                    for (int e = 0; e < 8; ++e) kv[e] = static_cast<__bf16>(__builtin_fmaf(c8[e], sf[e], zf[e]));
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        s[v][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            kv, __builtin_bit_cast(bf16x8, q_bf[nb * 16 + qn][g * (D / 32) + j]), s[v][nb], 0,
                            0, 0);
                }
            }
        } else {
            uint4 kr[2][KS];
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const int token = t0 + 8 * (n >> 2) + 4 * v + (n & 3);
                const uint16_t* src = p.k_ring + (static_cast<int64_t>(c.b) * p.kv_heads + c.kvh) * p.ring * D +
                                      static_cast<int64_t>(token % p.ring) * D + g * (D / 4);
#pragma unroll
                for (int j = 0; j < KS; ++j) kr[v][j] = *reinterpret_cast<const uint4*>(src + 8 * j);
            }
            if (kJointRing && value_ring) load_value_ring();
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the ring loads of this rare branch
#pragma unroll
            for (int v = 0; v < 2; ++v)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int j = 0; j < KS; ++j)
                        s[v][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, kr[v][j]),
                            __builtin_bit_cast(bf16x8, q_bf[nb * 16 + qn][g * (D / 32) + j]), s[v][nb], 0, 0, 0);
        }
        // scores in log2 units; masking where the tile holds a row's end, a causal limit or a missing page
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[v][nb][i] *= score_scale;
        if (p.softcap > 0.0f) {
            const float inv_cap = 1.0f / p.softcap;
#pragma unroll
            for (int v = 0; v < 2; ++v)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[v][nb][i] = soft_cap_log2(s[v][nb][i], p.softcap, inv_cap);
        }
        if (t0 + KPAGE > all_see || (!valid && t0 < kq) || p.mask) {
#pragma unroll
            for (int v = 0; v < 2; ++v)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int token = t0 + 8 * g + 4 * v + i;
                        bool ok = static_cast<float>(token) < limit[nb] && (valid || token >= kq);
                        if (p.mask) ok = ok && ((tile.mw[nb] >> (4 * v + i)) & 1u);
                        s[v][nb][i] = ok ? s[v][nb][i] : -INFINITY;
                    }
        }
        // online softmax with lazy rescaling (the reference maximum moves when a score exceeds it by 2^8)
        float pw[NB][8];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            float tile_max = -INFINITY;
#pragma unroll
            for (int v = 0; v < 2; ++v)
                tile_max = max_nan(max_nan(tile_max, max_nan(s[v][nb][0], s[v][nb][1])),
                                   max_nan(s[v][nb][2], s[v][nb][3]));
            // the ballot sees every lane's own maximum, so only a rescale needs the maximum over the lane group
            if (__ballot(tile_max > m_i[nb] + 8.0f || m_i[nb] == -INFINITY) != 0) {
                const bool fresh = m_i[nb] == -INFINITY;
                const float m_new = fmaxf(m_i[nb], group_max(tile_max));
                const float alpha = fresh ? 0.0f : __builtin_amdgcn_exp2f(m_i[nb] - m_new);
                l_i[nb] *= alpha;
#pragma unroll
                for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[nd][nb][i] = fresh ? 0.0f : acc[nd][nb][i] * alpha;
                m_i[nb] = m_new;
            }
            const float neg_m = m_i[nb] == -INFINITY ? 0.0f : -m_i[nb];
            float sum = 0.0f;
#pragma unroll
            for (int v = 0; v < 2; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pw[nb][4 * v + i] = __builtin_amdgcn_exp2f(s[v][nb][i] + neg_m);
                    sum += pw[nb][4 * v + i];
                }
            l_i[nb] += sum;  // the lane's own tokens; summed over the lane group at the end of the segment
        }
        // values: element e of the lane's operands is token t0 + 8 g + e; p as bf16 hi + lo for both sources (p is
        // zero at every token that no query row sees)
        bf16x8 phi[NB], plo[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) split_bf16(pw[nb], phi[nb], plo[nb]);
        auto product = [&](int nd, uint4 a4) __attribute__((always_inline)) {
            const bf16x8 a = __builtin_bit_cast(bf16x8, a4);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, phi[nb], acc[nd][nb], 0, 0, 0);
                acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, plo[nb], acc[nd][nb], 0, 0, 0);
            }
        };
        if (t0 < vq) {  // from codes: O += bf16(c * s + z) . p
            // tokens at or past vq and every token of a missing page are zero (an unwritten scale may be inf or
            // NaN); a tile of codes only skips the masks
            auto from_codes = [&](auto full_tag, const HalfMask& mask) __attribute__((always_inline)) {
                constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
                for (int nd = 0; nd < ND; ++nd) {
                    const int at = ((nd / 2) * 32 + 8 * g) * 2;
                    const uint4 v = dequant_values<BITS>(tile.vc[nd], g, *reinterpret_cast<const uint4*>(sl + 4 * D + at),
                                                         *reinterpret_cast<const uint4*>(sl + 6 * D + at));
                    product(nd, kFull ? v : apply_mask(v, mask));
                }
            };
            if (NB <= 2 && t0 + KPAGE <= vq && valid) {  // (at four column blocks the second copy would spill)
                from_codes(std::integral_constant<bool, NB <= 2>{}, HalfMask{});
            } else {
                from_codes(std::false_type{}, half_mask(code_values(tile, t0)));
            }
        }
        if (value_ring) {  // from the ring (tokens at or past vq, below the row's end)
            const int from = max(vq - tok0, 0), to = min(row_len - tok0, 8);
            const uint32_t keep = to > from ? ((to >= 8 ? 0xFFu : (1u << to) - 1u) & ~((1u << from) - 1u)) : 0u;
            const HalfMask mask = half_mask(keep);
            if (!kJointRing || !key_ring) {
                load_value_ring();
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the ring loads of this rare branch
            }
#pragma unroll
            for (int nd = 0; nd < ND; ++nd) product(nd, apply_mask(vr[nd], mask));
        }
    };

    // ---- end of a row segment: direct output, or a partial and (for the last wave of the row) the merge ----
    auto finish = [&](const Cursor& c, int64_t seg_begin, int64_t seg_end, bool first_segment) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) l_i[nb] = group_sum(l_i[nb]);
        const auto& o = acc;
        const int64_t row_end = c.row_start + c.row.tiles;
        if (seg_begin == c.row_start && seg_end == row_end) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int r = row0 + nb * 16 + n;
                if (r >= p.rows) continue;
#pragma unroll
                for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        store_output(p, c.b, c.kvh, r, 16 * nd + 4 * g + i, o[nd][nb][i], m_i[nb], l_i[nb]);
            }
            return;
        }
        if constexpr (kSplit) {
            // the second piece overwrites the query rows: no LDS access of the tile may move past this point
            if (!first_segment) __asm__ volatile("" ::: "memory");
            write_piece(pieces, 2 * wave + (first_segment ? 0 : 1), c, p.rows, n, g, lane, m_i[0], l_i[0],
                        [&](int nd, int i) __attribute__((always_inline)) { return o[nd][0][i]; });
            return;
        }
        const int64_t stride = static_cast<int64_t>(p.rows) * (D + 2);
        float* slot = p.part + (2 * static_cast<int64_t>(w) + (first_segment ? 0 : 1)) * stride;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int r = row0 + nb * 16 + n;
            if (r >= p.rows) continue;
            if (g == 0) {
                coherent_store(slot + r, m_i[nb]);
                coherent_store(slot + p.rows + r, l_i[nb]);
            }
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    coherent_store(slot + 2 * p.rows + r * D + 16 * nd + 4 * g + i, o[nd][nb][i]);
        }
        hand_off<D>(p, c, total, grid, lane);
    };

    // ---- the tile pipeline (as in paged_attention.hip) ----
    auto pipeline = [&]() __attribute__((always_inline)) {
        Cursor cur = small ? locate_in(p, rt, lo) : locate(p, lo, lane);
        PageWindow win;
        int64_t seg_begin = lo;
        bool first_segment = true;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int nd = 0; nd < ND; ++nd) acc[nd][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        begin_row(cur);

        // with two buffers a tile's loads are issued a tile ahead
        T bufs[NBUF];
        Cursor cs[NBUF];
        Cursor icur = cur;
        int64_t ipos = lo;
        auto issue_next = [&](T& buf, Cursor& slot) __attribute__((always_inline)) {
            issue_tile<D, BITS>(p, at_tile(icur), n, g, lane, win, buf);
            if (p.mask)  // the tile is one page: its word of every query row's mask
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    buf.mw[nb] = (mask_word(p, icur.b, icur.kvh, row0 + nb * 16 + n, at_tile(icur).t) >> (8 * g)) & 0xFFu;
            slot = icur;
            if (ipos < hi) {
                if (ipos + 1 < hi) advance(p, icur, small ? &rt : nullptr);
                ++ipos;
            }
        };
#pragma unroll
        for (int s = 0; s + 1 < NBUF; ++s) issue_next(bufs[s], cs[s]);

        int64_t pos = lo;
        auto step = [&](auto tag) __attribute__((always_inline)) -> bool {
            constexpr int I = decltype(tag)::value;
            constexpr int J = (I + NBUF - 1) % NBUF;
            issue_next(bufs[J], cs[J]);
            cur = cs[I];
            if (cur.t == 0 && pos != lo) begin_row(cur);
            compute(bufs[I], cur);
            const bool more = pos + 1 < hi;
            if (cur.t + 1 == cur.row.tiles || !more) {
                finish(cur, seg_begin, pos + 1, first_segment);
                first_segment = false;
                seg_begin = pos + 1;
            }
            ++pos;
            return more;
        };
        if constexpr (NBUF == 1) {
            while (step(std::integral_constant<int, 0>{})) {
            }
        } else {
            static_assert(NBUF == 2, "one or two tile buffers");
            while (step(std::integral_constant<int, 0>{}) && step(std::integral_constant<int, 1>{})) {
            }
        }
    };
    if constexpr (!kSplit) {
        pipeline();
    } else {
        if (lo < hi) pipeline();
        merge_pieces<D, WAVES>(p, pieces, wave, lane, wlo, whi, total, grid, w);
    }
}

// ---- host side ----------------------------------------------------------------------------------------------

namespace {

// Tile buffers of the one-column-block instances (ECO_KIVI_STAGES = 1 or 2 overrides): at D = 128 two (the next
// tile's loads in flight; two waves per SIMD since a tile's scales pass through LDS: int4 63-64 us against 65-67 us
// with one buffer at B=16, L=8192), at D = 64 one (three waves per SIMD).
int kivi_stages(int head_dim) {
    static const int forced = [] {
        const char* env = std::getenv("ECO_KIVI_STAGES");
        const int v = env ? std::atoi(env) : 0;
        return v <= 0 ? 0 : (v == 1 ? 1 : 2);
    }();
    return forced ? forced : (head_dim == 128 ? 2 : 1);
}

// Column blocks of 16 query rows from which the verification kernel (kivi_verify.hip: two-page tiles shared by four
// waves) serves (default 3: more than 32 query rows per KV head); ECO_KIVI_SHARED overrides.
int kivi_shared_from() {
    static const int from = [] {
        const char* env = std::getenv("ECO_KIVI_SHARED");
        const int v = env ? std::atoi(env) : 3;
        return v < 2 ? 2 : v;
    }();
    return from;
}

// An attention instance: the kernel, its threads per workgroup and the parts a workgroup's tile range is split in
// (the grid gives every part at least four tiles).
using KiviKernelFn = decltype(&kivi_attention_kernel<64, 2, 1, 1, 16>);
struct KiviInstance {
    KiviKernelFn kernel;
    int threads;
    int parts;
};

template <int D, int BITS, int NB, int NBUF, int PR>
KiviInstance kivi_instance() {
    constexpr int waves = kivi_wg_waves<D, NB>();
    return {kivi_attention_kernel<D, BITS, NB, NBUF, PR>, 64 * waves, waves};
}

// NB column blocks of query rows below kivi_shared_from(): one block, the split instance (one or two tile buffers,
// pieces of PR rows); otherwise one wave over NB blocks.
template <int D, int BITS, int NB, int PR>
KiviInstance kivi_kernel_of() {
    if constexpr (NB == 1)
        return kivi_stages(D) == 1 ? kivi_instance<D, BITS, 1, 1, PR>() : kivi_instance<D, BITS, 1, 2, PR>();
    return kivi_instance<D, BITS, NB, 1, 16>();
}

template <typename F>
int kivi_dispatch(int head_dim, int bits, int rows, const F& f) {
    const int nb = (rows + 15) / 16;
    auto by_nb = [&](auto d_tag, auto b_tag) -> int {
        constexpr int D = decltype(d_tag)::value;
        constexpr int BITS = decltype(b_tag)::value;
        if (nb == 1) {
            if (rows <= 4) return f.template run<D, BITS, 1, 4>();
            if (rows <= 8) return f.template run<D, BITS, 1, 8>();
            return f.template run<D, BITS, 1, 16>();
        }
        if (nb == 2) return f.template run<D, BITS, 2, 16>();
        if (nb <= 4) return f.template run<D, BITS, 4, 16>();
        return fail("kivi decode attention takes at most 64 query rows per KV head");
    };
    auto by_bits = [&](auto d_tag) -> int {
        if (bits == 2) return by_nb(d_tag, std::integral_constant<int, 2>{});
        if (bits == 4) return by_nb(d_tag, std::integral_constant<int, 4>{});
        return fail("kivi decode attention supports 2- and 4-bit codes");
    };
    if (head_dim == 64) return by_bits(std::integral_constant<int, 64>{});
    if (head_dim == 128) return by_bits(std::integral_constant<int, 128>{});
    return fail("kivi decode attention supports head dims 64 and 128");
}

struct KiviLaunch {
    hipStream_t stream;
    const KiviParams* p;
    template <int D, int BITS, int NB, int PR>
    int run() const {
        if (NB >= kivi_shared_from()) return kivi_verify_attention(*p, stream);
        const KiviInstance in = kivi_kernel_of<D, BITS, NB, PR>();
        hipLaunchKernelGGL(in.kernel, dim3(p->grid), dim3(in.threads), 0, stream, *p);
        return check_launch("kivi_attention_kernel");
    }
};

struct KiviOccupancy {
    int* per_cu;
    int* waves;
    template <int D, int BITS, int NB, int PR>
    int run() const {
        if (NB >= kivi_shared_from()) {
            *waves = 2;  // two-page tiles: four tiles per workgroup are eight pages
            return kivi_verify_resident_groups(D, BITS, per_cu);
        }
        int blocks = 0;
        const KiviInstance in = kivi_kernel_of<D, BITS, NB, PR>();
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, in.kernel, in.threads, 0) != hipSuccess ||
            blocks <= 0)
            blocks = 1;
        *per_cu = blocks;
        *waves = in.parts;
        return 0;
    }
};

}  // namespace

int kivi_schedule(const int32_t* committed, int residual, int32_t* keys_quantized, int32_t* values_quantized,
                  int32_t* ranges, int batch, hipStream_t stream) {
    hipLaunchKernelGGL(kivi_schedule_kernel, dim3((batch + 255) / 256), dim3(256), 0, stream, committed, residual,
                       keys_quantized, values_quantized, ranges, batch);
    return check_launch("kivi_schedule_kernel");
}

int kivi_ring_write(const KiviRingParams& p, hipStream_t stream) {
    if (p.tokens == 0) return 0;
    hipLaunchKernelGGL(kivi_ring_kernel, dim3(p.tokens), dim3(256), 0, stream, p);
    return check_launch("kivi_ring_kernel");
}

int kivi_quantize(const KiviQuantParams& p, int kind, int max_tokens, hipStream_t stream) {
    const int pages = (max_tokens + KPAGE - 1) / KPAGE + 1;  // a range need not start at a page boundary
    dim3 grid(p.batch * p.kv_heads, pages);
    if (kind == 0)
        hipLaunchKernelGGL(kivi_quant_keys_kernel, grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(kivi_quant_values_kernel, grid, dim3(256), 0, stream, p);
    return check_launch(kind == 0 ? "kivi_quant_keys_kernel" : "kivi_quant_values_kernel");
}

int kivi_resident_groups(int head_dim, int bits, int rows, int* per_cu, int* waves) {
    return kivi_dispatch(head_dim, bits, rows, KiviOccupancy{per_cu, waves});
}

int kivi_attention(const KiviParams& p, hipStream_t stream) {
    return kivi_dispatch(p.head_dim, p.bits, p.rows, KiviLaunch{stream, &p});
}

}  // namespace eco
