// Decode attention over a paged fp8 / bf16 KV cache on CDNA4 matrix cores (gfx950), one launch per call.
//
// What it computes is the reference's decode attention (attention/decode.py:66-103 as the definition,
// attention/_decode_kernels.py:110-226 for the log2-unit online softmax and the log-sum-exp merge of partial
// results): for every batch row b, KV head kvh and query row r = g * Q + qi of its group (query head
// h = kvh * G + g),
//   out[b, qi, h] = sum_t softmax_t(q . k_t * scale) v_t   over the row's visible tokens,
// with K/V decoded exactly from fp8 and multiplied by per-head scales. A page list turns it into Quest's gathered
// attention (attention/_quest_kernels.py:13-97): the virtual key axis is the selected pages, then the dense tail.
//
// Cache layout (vLLM's paged-attention layout, 16-token pages):
//   keys   [pages, Hkv, D / X, 16, X]  (X = 16 bytes of channels: 16 fp8 or 8 bf16)
//   values [pages, Hkv, D, 16]         (a channel's 16 tokens contiguous)
//
// Work decomposition (stream-K over waves). The work is the sequence of tiles (4 virtual pages = 64 tokens) of
// every (b, kvh) row, rows in (b, kvh) order. Each single-wave workgroup w of the G launched takes the contiguous
// range [W w / G, W (w + 1) / G) of the W tiles, so every wave streams the same number of bytes whatever the row
// lengths are. A row that lies inside one wave's range is finished by that wave and written directly; a row cut by
// range boundaries is left as partial (max, sum, acc) results in the workspace (at most two per wave: its first and
// its last row) and the last of its waves to finish (a per-row counter) merges them. Tile loads are double-buffered
// where the registers allow: the next tile's K/V (and at a row change its query) are in flight while the current
// tile is computed.
//
// Per tile a wave computes S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (M = 16 tokens, N = 16 query rows, K = 32
// channels) and O^T += V^T P^T (M = 16 channels, N = 16 query rows, K = 32 tokens):
//   * lane (n = l % 16, g = l / 16) holds A-row n and B-column n; the C/D fragment gives lane (n, g) rows 4g..4g+3.
//   * S MFMA v (v = 0..3) maps A-row m to token 4v + m % 4 of tile page m / 4, so lane group g ends with all 16
//     scores of page g for its query row (column n).
//   * the V operand of lane (n, g) is then channel n of page g: 16 (fp8) or 32 (bf16) contiguous bytes, one
//     vector load, and the scores it multiplies are already in the lane's registers (no cross-lane transpose).
//   * K is loaded as 16-byte runs: lane (n, g) reads run 4u + g of its token; the channel order this gives to the
//     MFMA's K dimension is mirrored in the query operand (a dot product does not depend on the order).
// fp8 bytes are converted exactly (v_cvt_scalef32_pk_{bf16,f16}_{fp8,bf8}, scale 1): keys to bf16 for S (the
// query is bf16, so every product is exact in the fp32 accumulator, as in the reference's tl.dot), values to fp16 for
// O with the softmax weights P in fp16 (11 significant bits against the reference's bf16 rounding of P). A bf16
// cache multiplies its bf16 values by P split into two bf16 terms (P = P_hi + P_lo), two MFMAs per block.

#pragma once

#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "paged_attention.hpp"
#include "stream_k.hpp"

namespace eco {

namespace {

constexpr int PAGE = PagedParams::kPage;
constexpr int TILE = PagedParams::kTile;

template <int FMT, bool HIGH>
__device__ inline uint32_t fp8x2_to_bf16x2(uint32_t word) {
    bf16x2 r;
    if constexpr (FMT == FP8_E4M3)
        r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, HIGH);
    else
        r = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(word, 1.0f, HIGH);
    return __builtin_bit_cast(uint32_t, r);
}

// 8 fp8 bytes (two dwords) -> 8 bf16 (an MFMA operand).
template <int FMT>
__device__ inline bf16x8 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
    uint4 r;
    r.x = fp8x2_to_bf16x2<FMT, false>(lo);
    r.y = fp8x2_to_bf16x2<FMT, true>(lo);
    r.z = fp8x2_to_bf16x2<FMT, false>(hi);
    r.w = fp8x2_to_bf16x2<FMT, true>(hi);
    return __builtin_bit_cast(bf16x8, r);
}

template <int FMT, bool HIGH>
__device__ inline uint32_t fp8x2_to_f16x2(uint32_t word) {
    f16x2 r;
    if constexpr (FMT == FP8_E4M3)
        r = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, HIGH);
    else
        r = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(word, 1.0f, HIGH);
    return __builtin_bit_cast(uint32_t, r);
}

// 8 fp8 bytes -> 8 fp16 (exact: both fp8 formats are subsets of fp16).
template <int FMT>
__device__ inline f16x8 fp8x8_to_f16x8(uint32_t lo, uint32_t hi) {
    uint4 r;
    r.x = fp8x2_to_f16x2<FMT, false>(lo);
    r.y = fp8x2_to_f16x2<FMT, true>(lo);
    r.z = fp8x2_to_f16x2<FMT, false>(hi);
    r.w = fp8x2_to_f16x2<FMT, true>(hi);
    return __builtin_bit_cast(f16x8, r);
}

__device__ inline uint32_t pack_f16x2(float a, float b) {
    f16x2 h = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
    return __builtin_bit_cast(uint32_t, h);
}

__device__ inline uint32_t pack_bf16x2(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// A tile's 16-byte K/V load: nontemporal (streamed) where the call reads whole rows; plain for Quest's page lists,
// whose few tiles per wave are latency-bound (measured at the Quest workload: 61 us per call with streamed loads
// against 50 us plain).
template <bool NT>
__device__ inline uint4 load16(const uint8_t* p) {
    if constexpr (NT) return stream_load16(p);
    return *reinterpret_cast<const uint4*>(p);
}

// First channel of k-step j (8 channels) for lane group g: run 4u + g of E channels, half h of it.
template <int E>
__device__ constexpr int k_channel(int j, int g) {
    constexpr int per_run = E / 8;
    return E * (4 * (j / per_run) + g) + 8 * (j % per_run);
}

// A tile's K/V registers, and (unless RQ) the query operand of its row. With RQ the kernel keeps the query operand
// once per row instead (loaded with the row's first tile), which frees NB * D / 8 VGPRs per tile buffer.
template <int D, int FMT, int NB, bool RQ = false>
struct Tile {
    static constexpr int ES = FMT == BF16 ? 2 : 1;  // bytes per element
    static constexpr int NU = D * ES / 64;          // 16-byte K loads per lane per S MFMA block
    static constexpr int ND = D / 16;               // value blocks of 16 channels
    static constexpr int NV = ES;                   // 16-byte V loads per lane per value block
    static constexpr int KS = D / 32;               // k-steps of an S MFMA block
    uint4 k[4][NU];
    uint4 v[ND][NV];
    bf16x8 q[RQ ? 1 : NB][RQ ? 1 : KS];  // the query operand of the tile's row (an L2 hit after the row's first tile)
    int lv;    // logical page of the lane group's tile page (-1: none)
    int vcnt;  // tokens of that page inside the row (0 to 16); the V bytes of the others are cleared before use
    uint32_t mw[NB];  // with a mask: bit k = token lv * 16 + k of query row nb * 16 + n is visible
};

// The mask bits of the lane group's tile page for each column block (loaded only with a mask).
template <int D, int FMT, int NB, bool RQ>
__device__ __forceinline__ void load_mask_bits(const PagedParams& p, const Cursor& c, int n, Tile<D, FMT, NB, RQ>& tile) {
    if (!p.mask) return;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
        tile.mw[nb] = tile.lv >= 0 ? mask_word(p, c.b, c.kvh, nb * 16 + n, tile.lv >> 1) >> (16 * (tile.lv & 1)) : 0u;
}

// The query operand of row c: lane (n, g) holds query row nb * 16 + n, channels of k-step j as the K runs order them
// (a lane of a row past the group reads row 0: its MFMA column is computed and never stored).
template <int D, int FMT, int NB>
__device__ __forceinline__ void load_query(const PagedParams& p, const Cursor& c, int n, int g,
                                           bf16x8 (&q)[NB][D / 32]) {
    constexpr int E = FMT == BF16 ? 8 : 16;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int r = nb * 16 + n;
        const bool valid = r < p.rows;
        const int gq = valid ? r / p.queries : 0;
        const int qi = valid ? r % p.queries : 0;
        const uint16_t* base = p.q + c.b * p.sq_b + qi * p.sq_q + (c.kvh * p.groups + gq) * p.sq_h;
#pragma unroll
        for (int j = 0; j < D / 32; ++j)
            q[nb][j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + k_channel<E>(j, g)));
    }
}

// The K/V loads of the tile at window offset `at`. K is read page-major: for tile page v, lane (n, g) loads token n,
// runs 4 u + g (one page per load instruction, four runs of 256 contiguous bytes: whole 128-byte lines; a mapping
// that put four pages in one instruction read half lines and streamed 2.5 us slower over the fp8 Llama-3-8B decode
// shape, 42.1 against 39.6 us for the loads alone). V: lane (n, g) loads channels 16 nd + n of tile page g. A page
// that holds nothing reads page 0 (its scores and values are masked when the tile is computed), and so does a dummy
// issue past the end of a wave's range: every path issues the same loads.
template <int D, int FMT, int NB, bool RQ, bool NT>
__device__ __forceinline__ void issue_kv(const PagedParams& p, const Cursor& c, int n, int g, int at,
                                         const PageWindow& win, Tile<D, FMT, NB, RQ>& tile, bool dummy) {
    using T = Tile<D, FMT, NB, RQ>;
    const int pv = dummy ? 0 : __shfl(win.physical, at + g);
    tile.lv = __shfl(win.logical, at + g);
    tile.vcnt = tile.lv >= 0 ? min(max(c.row.len - tile.lv * PAGE, 0), PAGE) : 0;
    load_mask_bits(p, c, n, tile);
    const uint8_t* kh = p.k_cache + c.kvh * p.kc_head;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int pk = dummy ? 0 : __builtin_amdgcn_readlane(win.physical, at + v);
        const uint8_t* kp = kh + static_cast<int64_t>(pk >= 0 ? pk : 0) * p.kc_page;
#pragma unroll
        for (int u = 0; u < T::NU; ++u) tile.k[v][u] = load16<NT>(kp + ((4 * u + g) * PAGE + n) * 16);
    }
    const uint8_t* vp = p.v_cache + c.kvh * p.vc_head + static_cast<int64_t>(pv >= 0 ? pv : 0) * p.vc_page;
#pragma unroll
    for (int nd = 0; nd < T::ND; ++nd)
#pragma unroll
        for (int w = 0; w < T::NV; ++w) tile.v[nd][w] = load16<NT>(vp + (16 * nd + n) * PAGE * T::ES + 16 * w);
}

// Issues the loads of the tile under cursor c and the query operand of its row into the tile.
template <int D, int FMT, int NB, bool NT>
__device__ __forceinline__ void issue_tile(const PagedParams& p, const Cursor& c, int n, int g, int lane, PageWindow& win,
                                  Tile<D, FMT, NB>& tile, bool dummy) {
    using T = Tile<D, FMT, NB>;
    ensure_window(p, c, lane, win);
    issue_kv<D, FMT, NB, false, NT>(p, c, n, g, TILE * c.t - win.base, win, tile, dummy);
    // the query operand: lane (n, g) holds query row nb * 16 + n, channels of k-step j as the K runs order them (a lane
    // of a row past the group reads row 0: its MFMA column is computed and never stored)
    constexpr int E = 16 / T::ES;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int r = nb * 16 + n;
        const bool valid = r < p.rows;
        const int gq = valid ? r / p.queries : 0;
        const int qi = valid ? r % p.queries : 0;
        const uint16_t* base = p.q + c.b * p.sq_b + qi * p.sq_q + (c.kvh * p.groups + gq) * p.sq_h;
#pragma unroll
        for (int j = 0; j < T::KS; ++j)
            tile.q[nb][j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + k_channel<E>(j, g)));
    }
}

// As issue_tile for a tile without a query operand: the row's query operand goes to q_next, only when load_q is set
// (the first tile of a row, or of the wave's range), and those loads come first, so that waiting for them does not
// wait for the tile's K/V.
template <int D, int FMT, int NB, bool NT>
__device__ __forceinline__ void issue_tile_rq(const PagedParams& p, const Cursor& c, int n, int g, int lane,
                                              PageWindow& win, Tile<D, FMT, NB, true>& tile,
                                              bf16x8 (&q_next)[NB][D / 32], bool load_q, bool dummy) {
    if (load_q) load_query<D, FMT, NB>(p, c, n, g, q_next);
    ensure_window(p, c, lane, win);
    issue_kv<D, FMT, NB, true, NT>(p, c, n, g, TILE * c.t - win.base, win, tile, dummy);
}

// The 4 x 4 transpose of dword blocks over the lane rows (16 lanes each): row g's x[v] becomes row v's x[g], that is
// after the call row g holds in x[v] what row v held in x[g]. Two stages of lane swaps (the upper and lower 32
// lanes, then odd and even rows).
__device__ __forceinline__ void transpose_rows4(uint32_t (&x)[4]) {
    const auto a = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    x[0] = c[0];
    x[1] = c[1];
    x[2] = d[0];
    x[3] = d[1];
}

// Clears the V bytes of the tokens a tile page does not hold (past the row's end, or the whole page when it holds
// nothing): cache slots that were never written may hold NaN codes, and a zero softmax weight times NaN is NaN.
// V run w of a lane holds 16 bytes of channel data for tokens 16 w / ES .. of its page (ES bytes per token).
template <int D, int FMT, int NB, bool RQ>
__device__ inline void clear_unheld_values(Tile<D, FMT, NB, RQ>& tile) {
    using T = Tile<D, FMT, NB, RQ>;
    constexpr int TPD = 4 / T::ES;  // tokens per dword
    uint32_t mask[T::NV][4];
#pragma unroll
    for (int w = 0; w < T::NV; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int first = (4 * w + i) * TPD;  // first token of this dword
            const int held = min(max(tile.vcnt - first, 0), TPD);
            mask[w][i] = held == TPD ? 0xFFFFFFFFu : (1u << (8 * T::ES * held)) - 1u;
        }
#pragma unroll
    for (int nd = 0; nd < T::ND; ++nd)
#pragma unroll
        for (int w = 0; w < T::NV; ++w) {
            tile.v[nd][w].x &= mask[w][0];
            tile.v[nd][w].y &= mask[w][1];
            tile.v[nd][w].z &= mask[w][2];
            tile.v[nd][w].w &= mask[w][3];
        }
}

}  // namespace

// Two waves per SIMD for the single-buffer instances whose state fits 256 VGPRs: the compiler then keeps the
// accumulators in VGPRs (no copies between the accumulation registers and the VGPRs at every tile), and the second
// wave's loads and arithmetic fill the first one's waits. These instances also clear the accumulators through a
// row's first rescale and take the soft cap through the hardware reciprocal (see begin_row and compute); the others
// keep the explicit clear and the IEEE divisions.
template <int D, int FMT, int NB, int NBUF>
constexpr int waves_per_simd() {
    return NBUF == 1 && D <= 128 && (NB == 1 || (NB == 2 && FMT != BF16)) ? 2 : 1;
}

// Waves of a workgroup. Four for one column block at D <= 128: the workgroup's tile range is split in four
// contiguous quarters, and the pieces of a row that lies inside the workgroup's range are merged through LDS after
// one barrier; only rows cut at a workgroup boundary go through the counter and the workspace partials.
template <int D, int FMT, int NB, int NBUF>
constexpr int wg_waves() {
    return NB == 1 && D <= 128 && NBUF <= 2 ? 4 : 1;
}

// QH: fp16 queries (an fp8 cache): the keys are converted to fp16 (exact for both fp8 formats) and S takes
// v_mfma_f32_16x16x32_f16, every product exact as with bf16 queries; the operand registers hold the query's raw bits
// either way.
template <int D, int FMT, int NB, int NBUF, bool NT, bool QH = false>
__global__ __launch_bounds__((64 * wg_waves<D, FMT, NB, NBUF>()))
    __attribute__((amdgpu_waves_per_eu(waves_per_simd<D, FMT, NB, NBUF>()))) void
paged_attention_kernel(PagedParams p) {
    static_assert(!QH || FMT != BF16, "fp16 queries read an fp8 cache");
    constexpr bool kTwoWaves = waves_per_simd<D, FMT, NB, NBUF>() == 2;
    constexpr int WAVES = wg_waves<D, FMT, NB, NBUF>();
    // two buffers: the query operand is kept once per row (q_row), loaded into q_next with the row's first tile
    constexpr bool kRowQ = NBUF == 2;
    using T = Tile<D, FMT, NB, kRowQ>;
    constexpr int ES = T::ES;
    constexpr int E = 16 / ES;  // channels per 16-byte run
    constexpr int KS = D / 32;  // k-steps of an S MFMA block
    constexpr int ND = T::ND;
    constexpr int KPR = E / 8;  // k-steps per run

    const int lane = WAVES > 1 ? static_cast<int>(threadIdx.x) & 63 : static_cast<int>(threadIdx.x);
    const int wave = WAVES > 1 ? uniform(static_cast<int>(threadIdx.x) >> 6) : 0;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int w = xcd_range(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));  // the workgroup's range
    const int grid = gridDim.x;

    // row geometry: one load of the lengths for batches of at most 64 rows
    const bool small = p.batch <= 64;
    RowTable rt{};
    if (small) rt = row_table(p, lane);
    const int64_t total = small ? uniform64(__shfl(rt.incl, 63)) : uniform64(total_tiles(p, lane));
    // rows of batch entries without a key: zeros (sinks included, decode.py:17)
    for (int b = w * WAVES + wave; b < p.batch; b += grid * WAVES) {
        if ((small ? __builtin_amdgcn_readlane(rt.row.tiles, b) : row_of(p, b).tiles) == 0)
            for (int idx = lane; idx < p.kv_heads * p.rows * D; idx += 64)
                store_output(p, b, idx / (p.rows * D), (idx / D) % p.rows, idx % D, 0.0f, -INFINITY, 0.0f);
    }
    const int64_t wlo = total * w / grid;  // the workgroup's tile range
    const int64_t whi = total * (w + 1) / grid;
    const int64_t lo = wlo + (whi - wlo) * wave / WAVES;  // this wave's quarter of it
    const int64_t hi = wlo + (whi - wlo) * (wave + 1) / WAVES;
    // row pieces of the workgroup's waves (stream_k.hpp)
    __shared__ typename std::conditional<(WAVES > 1), Pieces<D, WAVES>, char>::type pieces;
    if constexpr (WAVES > 1) {
        clear_pieces(pieces, wave, lane);
    } else {
        if (lo >= hi) return;
    }

    // ---- row state: query operand, visibility limits, scales, online-softmax accumulators ----
    float limit[NB];
    int all_see = 0;  // tokens below this are visible to every query row of the row
    float score_scale = 0.0f, vs = 1.0f;
    float m_i[NB], l_i[NB];  // l_i: the sum over the lane's own tokens until the segment's end reduces it
    f32x4 acc[ND][NB];

    auto begin_row = [&](const Cursor& c) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int r = nb * 16 + n;
            limit[nb] = r < p.rows ? static_cast<float>(c.row.len - p.queries - p.queries_after + r % p.queries + 1) : 0.0f;
            m_i[nb] = -INFINITY;
            l_i[nb] = 0.0f;
            // two-wave instances: the accumulators are cleared by the row's first rescale (m_i = -inf marks a row
            // with no weight yet), so that a row change does not give them a second register version to merge at
            // every tile
            if constexpr (!kTwoWaves)
#pragma unroll
                for (int nd = 0; nd < ND; ++nd) acc[nd][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        all_see = c.row.len - p.queries - p.queries_after + 1;
        const float ks = p.k_scale ? scalar_load(p.k_scale, c.kvh) : 1.0f;
        vs = p.v_scale ? scalar_load(p.v_scale, c.kvh) : 1.0f;
        score_scale = p.softcap > 0.0f ? p.scale * ks : p.scale * ks * kLog2e;
    };

    // ---- one tile of the online softmax ----
    bf16x8 q_row[kRowQ ? NB : 1][kRowQ ? KS : 1], q_next[kRowQ ? NB : 1][kRowQ ? KS : 1];
    auto compute = [&](T& tile) __attribute__((always_inline)) {
        if (__ballot(tile.vcnt < PAGE) != 0) clear_unheld_values<D, FMT, NB, kRowQ>(tile);
        f32x4 s[4][NB];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s[v][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const uint4 run = tile.k[v][j / KPR];
                bf16x8 a;
                f16x8 ah;
                if constexpr (FMT == BF16) {
                    a = __builtin_bit_cast(bf16x8, run);
                } else if constexpr (QH) {
                    const int h2 = j % KPR;
                    ah = fp8x8_to_f16x8<FMT>(h2 ? run.z : run.x, h2 ? run.w : run.y);
                } else {
                    const int h2 = j % KPR;
                    a = fp8x8_to_bf16x8<FMT>(h2 ? run.z : run.x, h2 ? run.w : run.y);
                }
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                {
                    bf16x8 qo;
                    if constexpr (kRowQ)
                        qo = q_row[nb][j];
                    else
                        qo = tile.q[nb][j];
                    if constexpr (QH)
                        s[v][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, __builtin_bit_cast(f16x8, qo), s[v][nb],
                                                                           0, 0, 0);
                    else
                        s[v][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qo, s[v][nb], 0, 0, 0);
                }
            }
        }
        // P operands: fp16 for fp8 caches, bf16 hi + lo for bf16 caches
        f16x8 pop_h[NB][2];
        bf16x8 pop_hi[NB][2], pop_lo[NB][2];
        const int first = tile.lv * PAGE;  // position of token 0 of tile page g
        // Scores in log2 units (times the scale, through the soft cap if one is set). Only a tile that holds a
        // row's end, an empty page or a token some causal query row must not see is masked, and every tile of a
        // call with a mask (visible = the causal limit and the mask bit).
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[v][nb][i] *= score_scale;
        if (p.softcap > 0.0f) {
            const float inv_cap = 1.0f / p.softcap;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if constexpr (kTwoWaves) {
                            s[v][nb][i] = soft_cap_log2(s[v][nb][i], p.softcap, inv_cap);
                        } else {
                            const float t = s[v][nb][i] / p.softcap;
                            const float e = __expf(-2.0f * fabsf(t));
                            const float th = (1.0f - e) / (1.0f + e);
                            s[v][nb][i] = p.softcap * (t < 0.0f ? -th : th) * kLog2e;
                        }
                    }
        }
        if (p.mask || __ballot(tile.lv < 0 || first + PAGE > all_see) != 0) {
            // score (v, i) of lane (n, g) is token 4 g + i of tile page v, whose logical page row v of the lanes holds
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int lv = __builtin_amdgcn_readlane(tile.lv, 16 * v);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const uint32_t bits = p.mask ? static_cast<uint32_t>(__shfl(static_cast<int>(tile.mw[nb]), 16 * v + n)) >> (4 * g) : 0u;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        bool ok = lv >= 0 && static_cast<float>(lv * PAGE + 4 * g + i) < limit[nb];
                        if (p.mask) ok = ok && ((bits >> i) & 1u);
                        s[v][nb][i] = ok ? s[v][nb][i] : -INFINITY;
                    }
                }
            }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            float tile_max = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; ++v)
                tile_max = max_nan(max_nan(tile_max, max_nan(s[v][nb][0], s[v][nb][1])),
                                   max_nan(s[v][nb][2], s[v][nb][3]));
            // Lazy rescaling: the reference maximum m_i moves only when a score exceeds it by more than 2^8, so that
            // the accumulators are rescaled a few times per row instead of at every tile (the weights stay below
            // 2^8, far inside fp16's range; the quotient acc / l does not depend on the reference). The ballot sees
            // every lane's own maximum; only a rescale needs the maximum over the lane group.
            constexpr float lazy = 8.0f;
            if constexpr (kTwoWaves) {
                if (__ballot(tile_max > m_i[nb] + lazy || m_i[nb] == -INFINITY) != 0) {
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
            } else if (__ballot(tile_max > m_i[nb] + lazy) != 0) {
                const float m_new = fmaxf(m_i[nb], group_max(tile_max));
                const float alpha = m_i[nb] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_i[nb] - m_new);
                l_i[nb] *= alpha;
#pragma unroll
                for (int nd = 0; nd < ND; ++nd) acc[nd][nb] *= alpha;
                m_i[nb] = m_new;
            }
            const float neg_m = m_i[nb] == -INFINITY ? 0.0f : -m_i[nb];
            float sum = 0.0f;
            float pw[4][4];
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pw[v][i] = __builtin_amdgcn_exp2f(s[v][nb][i] + neg_m);
                    sum += pw[v][i];
                }
            l_i[nb] += sum;
            // lane (n, g) holds the weights of tokens 4 g .. 4 g + 3 of every tile page; the P operand of lane (n, g)
            // is tile page g's 16 tokens (the page whose V channels it loads): a transpose of 4-token blocks over the
            // lane rows
            if constexpr (FMT == BF16) {
                uint32_t hi[2][4], lo[2][4];
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float x0 = pw[v][2 * h], x1 = pw[v][2 * h + 1];
                        hi[h][v] = pack_bf16x2(x0, x1);
                        lo[h][v] = pack_bf16x2(x0 - bits_f32(hi[h][v] << 16), x1 - bits_f32(hi[h][v] & 0xFFFF0000u));
                    }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    transpose_rows4(hi[h]);
                    transpose_rows4(lo[h]);
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    pop_hi[nb][u] = __builtin_bit_cast(bf16x8, make_uint4(hi[0][2 * u], hi[1][2 * u], hi[0][2 * u + 1], hi[1][2 * u + 1]));
                    pop_lo[nb][u] = __builtin_bit_cast(bf16x8, make_uint4(lo[0][2 * u], lo[1][2 * u], lo[0][2 * u + 1], lo[1][2 * u + 1]));
                }
            } else {
                uint32_t w[2][4];
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int h = 0; h < 2; ++h) w[h][v] = pack_f16x2(pw[v][2 * h], pw[v][2 * h + 1]);
#pragma unroll
                for (int h = 0; h < 2; ++h) transpose_rows4(w[h]);
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    pop_h[nb][u] = __builtin_bit_cast(f16x8, make_uint4(w[0][2 * u], w[1][2 * u], w[0][2 * u + 1], w[1][2 * u + 1]));
            }
        }
        // O^T += V^T P^T: lane (n, g) supplies channel 16 nd + n of tile page g
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if constexpr (FMT == BF16) {
                    const bf16x8 a = __builtin_bit_cast(bf16x8, tile.v[nd][u]);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pop_hi[nb][u], acc[nd][nb], 0, 0, 0);
                        acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pop_lo[nb][u], acc[nd][nb], 0, 0, 0);
                    }
                } else {
                    const uint4 run = tile.v[nd][0];
                    const f16x8 a = fp8x8_to_f16x8<FMT>(u ? run.z : run.x, u ? run.w : run.y);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pop_h[nb][u], acc[nd][nb], 0, 0, 0);
                }
            }
        }
    };

    // ---- end of a row segment: direct output, or a partial and (for the last wave of the row) the merge ----
    auto finish = [&](const Cursor& c, int64_t seg_begin, int64_t seg_end, bool first_segment) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) l_i[nb] = group_sum(l_i[nb]);
        const int64_t row_end = c.row_start + c.row.tiles;
        if (seg_begin == c.row_start && seg_end == row_end) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int r = nb * 16 + n;
                if (r >= p.rows) continue;
#pragma unroll
                for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        store_output(p, c.b, c.kvh, r, 16 * nd + 4 * g + i, acc[nd][nb][i] * vs, m_i[nb], l_i[nb]);
            }
            return;
        }
        if constexpr (WAVES > 1) {
            write_piece(pieces, 2 * wave + (first_segment ? 0 : 1), c, p.rows, n, g, lane, m_i[0], l_i[0],
                        [&](int nd, int i) __attribute__((always_inline)) { return acc[nd][0][i] * vs; });
            return;
        }
        const int64_t stride = static_cast<int64_t>(p.rows) * (D + 2);
        float* slot = p.part + (2 * static_cast<int64_t>(w) + (first_segment ? 0 : 1)) * stride;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int r = nb * 16 + n;
            if (r >= p.rows) continue;
            if (g == 0) {
                coherent_store(slot + r, m_i[nb]);
                coherent_store(slot + p.rows + r, l_i[nb]);
            }
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    coherent_store(slot + 2 * p.rows + r * D + 16 * nd + 4 * g + i, acc[nd][nb][i] * vs);
        }
        // the partial is released before the row's counter counts it; the last part acquires and merges them all
        hand_off<D>(p, c, total, grid, lane);
    };

    // ---- the tile pipeline: NBUF register buffers, tile pos + NBUF - 1 issued while tile pos is computed ----
    auto pipeline = [&]() __attribute__((always_inline)) {
        Cursor cur = small ? locate_in(p, rt, lo) : locate(p, lo, lane);
        PageWindow win;
        int64_t seg_begin = lo;
        bool first_segment = true;
        if constexpr (kTwoWaves)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int nd = 0; nd < ND; ++nd) acc[nd][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        begin_row(cur);

        T bufs[NBUF];
        Cursor cs[NBUF];  // the cursor of the tile each buffer holds
        Cursor icur = cur;  // the next tile to issue, at sequence offset ipos
        int64_t ipos = lo;

        // Every step issues one tile, past the end of the range a dummy that reads cache page 0 (never computed): with
        // the same number of loads issued on every path through the loop, the wait before a tile's use counts the
        // younger tiles' loads and leaves them in flight. (A branch around the issue, with a wait for every load on
        // the path that issues nothing, measured no faster at the fp8 Llama-3-8B decode shape and 4 us slower for
        // Quest's page lists.)
        auto issue_next = [&](T& buf, Cursor& slot) __attribute__((always_inline)) {
            const bool dummy = ipos >= hi;
            if constexpr (kRowQ)
                issue_tile_rq<D, FMT, NB, NT>(p, icur, n, g, lane, win, buf, q_next, icur.t == 0 || ipos == lo, dummy);
            else
                issue_tile<D, FMT, NB, NT>(p, icur, n, g, lane, win, buf, dummy);
            slot = icur;
            if (ipos < hi) {
                if (ipos + 1 < hi) advance(p, icur, small ? &rt : nullptr);
                ++ipos;
            }
        };
#pragma unroll
        for (int s = 0; s + 1 < NBUF; ++s) issue_next(bufs[s], cs[s]);

        int64_t pos = lo;
        // computes the tile held in buffer I (the loop is unrolled by NBUF so that every buffer index is a constant)
        auto step = [&](auto tag) __attribute__((always_inline)) -> bool {
            constexpr int I = decltype(tag)::value;
            constexpr int J = (I + NBUF - 1) % NBUF;
            if constexpr (kRowQ) {
                // the row's query operand moves to q_row before the next issue may reload q_next
                cur = cs[I];
                if (cur.t == 0 || pos == lo)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                        for (int j = 0; j < KS; ++j) q_row[nb][j] = q_next[nb][j];
                issue_next(bufs[J], cs[J]);
            } else {
                issue_next(bufs[J], cs[J]);
                cur = cs[I];
            }
            if (cur.t == 0 && pos != lo) begin_row(cur);
            compute(bufs[I]);
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
        } else if constexpr (NBUF == 2) {
            while (step(std::integral_constant<int, 0>{}) && step(std::integral_constant<int, 1>{})) {
            }
        } else {
            static_assert(NBUF == 3, "1 to 3 tile buffers");
            while (step(std::integral_constant<int, 0>{}) && step(std::integral_constant<int, 1>{}) &&
                   step(std::integral_constant<int, 2>{})) {
            }
        }
    };
    if constexpr (WAVES == 1) {
        pipeline();
    } else {
        if (lo < hi) pipeline();
        merge_pieces<D, WAVES>(p, pieces, wave, lane, wlo, whi, total, grid, w);
    }
}

}  // namespace eco
