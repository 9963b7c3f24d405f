// KIVI attention for many query rows per KV head (speculative verification: a draft of several tokens per row, the
// reference's kivi_decode_attention with Q > 1, attention/kivi.py:199-309 and its kernel _kivi_kernels.py) on gfx950.
//
// What it computes is kivi.hip's attention: keys and values dequantized as the reference does (bf16 of code * scale
// + zero, the product and the sum in fp32: one fused multiply-add, the product being exact), tokens not yet quantized
// read from the bf16 rings, scores on bf16 MFMAs, the value product's B operand p split into bf16 hi + lo, a causal
// limit per query row from the lengths (query qi of a row of length L sees tokens < L - Q + qi + 1) and the optional
// packed mask, sinks and a soft cap.
//
// Work decomposition: stream-K over tiles of 64 tokens (two cache pages; stream_k.hpp with two pages per tile), the
// four waves of a workgroup walking the workgroup's range together, wave w holding query rows 16 w .. 16 w + 15.
// Per tile, the workgroup's 256 lanes dequantize the tile once into LDS (keys row-major, values transposed so that a
// lane's 8 tokens of one channel are one 16-byte read), one barrier, then every wave computes its rows' scores
// (4 x D / 32 MFMAs), the online softmax and P.V (2 x 2 x D / 16 MFMAs) from LDS. The LDS tiles are double-buffered,
// so one barrier per tile also orders a buffer's reuse two tiles later; the next tile's codes, scales and zero points
// (a few registers per lane) are loaded while the current tile is computed. A row cut at workgroup boundaries leaves
// its segments' partials in the workspace and a second launch merges them: a partial here is 64 query rows wide, and
// the hand-off inside the kernel (stores waited for, counter, merge) stalled the tile pipeline of every workgroup
// (66 us of 226 at B=64, Q=8, L~U[1024, 4096]; the decode kernels keep it, their partials being a few rows).

#include <type_traits>

#include "common.hpp"
#include "kivi.hpp"
#include "kivi_math.hpp"
#include "stream_k.hpp"

namespace eco {

namespace {

// The stream-K geometry of this kernel: tiles of two 32-token pages.
struct VerifyParams : KiviParams {
    static constexpr int kTile = 2;
};

constexpr int VPAGE = KiviParams::kPage;  // tokens per cache page
constexpr int VTILE = 2 * VPAGE;          // tokens per tile

// A lane's share of a tile's loads. Keys: page pg = lane's wave / 2, channels 8 co .. 8 co + 7 of TPT tokens (one
// code word each, the scale and zero point of the 8 channels). Values: CPT channels of one value group, tokens
// 8 o .. 8 o + 7 (one code word each, the 8 tokens' scales and zero points of the group).
template <int D>
struct Share {
    static constexpr int TPT = D / 32;  // key tokens per lane
    static constexpr int CPT = D / 32;  // value channels per lane
    uint32_t kw[TPT];
    uint4 ks, kz;
    uint32_t vw[CPT];
    uint4 vs, vz;
    int page;  // physical page of the lane's page (the same in a wave), -1 for none
};

__device__ inline uint32_t half_keep(uint32_t keep, int j) {  // the bf16 halves of word j of a uint4 (bit e = element e)
    return ((keep >> (2 * j)) & 1u ? 0x0000FFFFu : 0u) | ((keep >> (2 * j + 1)) & 1u ? 0xFFFF0000u : 0u);
}

// Elements of a whose bit in keep is set, else those of b.
__device__ inline uint4 select8(uint32_t keep, uint4 a, uint4 b) {
    const uint32_t m0 = half_keep(keep, 0), m1 = half_keep(keep, 1), m2 = half_keep(keep, 2), m3 = half_keep(keep, 3);
    return make_uint4((a.x & m0) | (b.x & ~m0), (a.y & m1) | (b.y & ~m1), (a.z & m2) | (b.z & ~m2),
                      (a.w & m3) | (b.w & ~m3));
}

// bf16(code * scale + zero) of eight codes with their fp16 scales and zero points.
template <int BITS>
__device__ inline uint4 dequant8(uint32_t word, int h, const float (&sf)[8], const float (&zf)[8]) {
    float c8[8];
    codes_to_f32<BITS>(word, h, c8);
    bf16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<__bf16>(__builtin_fmaf(c8[i], sf[i], zf[i]));
    return __builtin_bit_cast(uint4, v);
}

__device__ inline void halves_to_f32(uint4 x, float (&out)[8]) {
    const f16x8 h = __builtin_bit_cast(f16x8, x);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(h[i]);
}

template <int D, int BITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void kivi_verify_kernel(VerifyParams p) {
    constexpr int KS = D / 32;           // k-steps of an S MFMA
    constexpr int ND = D / 16;           // value blocks of 16 channels
    constexpr int CO = D / 8;            // key channel octets
    constexpr int TPT = Share<D>::TPT;   // key tokens per lane
    constexpr int CPT = Share<D>::CPT;   // value channels per lane
    constexpr int KROW = 2 * D + 16;     // LDS bytes per key row (padded)
    constexpr int VROW = 2 * VTILE + 16;  // LDS bytes per transposed value row (one channel's 64 tokens, padded)
    constexpr KiviLayout L{D, BITS};
    __shared__ __align__(16) uint8_t kl[2][VTILE * KROW];
    __shared__ __align__(16) uint8_t vl[2][D * VROW];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int r = 16 * wave + n;  // the lane's query row (MFMA column n)
    const int w = xcd_range(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));  // the workgroup's range
    const int grid = gridDim.x;
    // the lane's dequantization items (pg is the same in a wave)
    const int pg = wave >> 1;
    const int rem = tid & 127;
    const int co = rem % CO, tg = rem / CO;    // keys: channels 8 co.., tokens TPT tg..
    const int vo = rem >> 5, cq = rem & 31;    // values: tokens 8 vo.., channels CPT cq..
    const int vgrp = (CPT * cq) / 32;          // their value group

    const bool small = p.batch <= 64;
    RowTable rt{};
    if (small) rt = row_table(p, lane);
    const int64_t total = small ? uniform64(__shfl(rt.incl, 63)) : uniform64(total_tiles(p, lane));
    for (int b = w * 4 + wave; b < p.batch; b += grid * 4) {  // rows without a key: zeros
        if ((small ? __builtin_amdgcn_readlane(rt.row.tiles, b) : row_of(p, b).tiles) == 0)
            for (int idx = lane; idx < p.kv_heads * p.rows * D; idx += 64)
                store_output(p, b, idx / (p.rows * D), (idx / D) % p.rows, idx % D, 0.0f, -INFINITY, 0.0f);
    }
    const int64_t lo = total * w / grid;  // the workgroup's tile range
    const int64_t hi = total * (w + 1) / grid;
    if (lo >= hi) return;  // (the same for every wave of the workgroup)

    // ---- row state ----
    int kq = 0, vq = 0, row_len = 0, all_see = 0;
    float limit = 0.0f, m_i = -INFINITY, l_i = 0.0f;
    bf16x8 qreg[KS];
    f32x4 acc[ND];
    auto begin_row = [&](const Cursor& c) __attribute__((always_inline)) {
        // query row r, channels g D / 4 + 8 j .. (the channel order of the key operand below); zero past the rows
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            uint4 x = make_uint4(0, 0, 0, 0);
            if (r < p.rows) {
                const int gq = r / p.queries, qi = r % p.queries;
                x = *reinterpret_cast<const uint4*>(p.q + c.b * p.sq_b + qi * p.sq_q + (c.kvh * p.groups + gq) * p.sq_h +
                                                    g * (D / 4) + 8 * j);
            }
            qreg[j] = __builtin_bit_cast(bf16x8, x);
        }
        // wait here for the query (vmcnt(0)), so that the tile steps, which load nothing of a row's own, do not wait at
        // this branch's join for every load in flight
        __builtin_amdgcn_s_waitcnt(0x0F70);
        kq = scalar_load(p.keys_quantized, c.b);
        vq = scalar_load(p.values_quantized, c.b);
        row_len = c.row.len;
        all_see = c.row.len - p.queries - p.queries_after + 1;
        limit = r < p.rows ? static_cast<float>(c.row.len - p.queries - p.queries_after + r % p.queries + 1) : 0.0f;
        m_i = -INFINITY;
        l_i = 0.0f;
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) acc[nd] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };
    const float score_scale = p.softcap > 0.0f ? p.scale : p.scale * kLog2e;

    // ---- the lane's loads of tile c (the same loads on every path: a missing page reads page 0) ----
    PageWindow win;
    auto issue = [&](Share<D>& s, const Cursor& c) __attribute__((always_inline)) {
        ensure_window(p, c, lane, win);
        const int phys = __builtin_amdgcn_readlane(win.physical, VerifyParams::kTile * c.t + pg - win.base);
        s.page = phys;
        const uint8_t* blk = p.blocks + static_cast<int64_t>(phys >= 0 ? phys : 0) * p.blk_page + c.kvh * p.blk_head;
        // codes, scales and zero points are read once per call: streamed loads
#pragma unroll
        for (int i = 0; i < TPT; ++i)
            s.kw[i] = __builtin_nontemporal_load(
                reinterpret_cast<const uint32_t*>(blk + L.k_codes() + (TPT * tg + i) * (D * BITS / 8)) +
                (BITS == 4 ? co : co / 2));
        s.ks = stream_load16(blk + L.k_scale() + 16 * co);
        s.kz = stream_load16(blk + L.k_zero() + 16 * co);
        const int u = BITS == 4 ? vo : vo >> 1;  // value word of tokens 8 vo ..
        const uint32_t* vwords = reinterpret_cast<const uint32_t*>(blk + L.v_codes());
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = CPT * cq + k;
            s.vw[k] = __builtin_nontemporal_load(vwords + (u * 16 + c % 16) * ND + c / 16);
        }
        s.vs = stream_load16(blk + L.v_scale() + (vgrp * 32 + 8 * vo) * 2);
        s.vz = stream_load16(blk + L.v_zero() + (vgrp * 32 + 8 * vo) * 2);
    };

    // ---- the lane's items of tile c into LDS buffer buf ----
    auto stage = [&](const Share<D>& s, const Cursor& c, int buf) __attribute__((always_inline)) {
        const int t0p = VTILE * c.t + VPAGE * pg;  // first token of the lane's page
        const int64_t row_kv = static_cast<int64_t>(c.b) * p.kv_heads + c.kvh;
        // keys: a page is all codes (below kq, whole key groups) or all ring; the scores of a missing codes page and
        // of tokens past the row are masked, so their entries need no care
        if (t0p < kq) {
            float sf[8], zf[8];
            halves_to_f32(s.ks, sf);
            halves_to_f32(s.kz, zf);
#pragma unroll
            for (int i = 0; i < TPT; ++i)
                *reinterpret_cast<uint4*>(kl[buf] + (VPAGE * pg + TPT * tg + i) * KROW + 16 * co) =
                    dequant8<BITS>(s.kw[i], BITS == 4 ? 0 : (co & 1), sf, zf);
        } else {
#pragma unroll
            for (int i = 0; i < TPT; ++i) {
                const int t = t0p + TPT * tg + i;
                *reinterpret_cast<uint4*>(kl[buf] + (VPAGE * pg + TPT * tg + i) * KROW + 16 * co) =
                    *reinterpret_cast<const uint4*>(p.k_ring + (row_kv * p.ring + t % p.ring) * D + 8 * co);
            }
        }
        // values: token t from codes below vq on a present page, from the ring in [vq, row_len), else zero (an
        // unwritten scale may be inf or NaN); a present page of codes only (the common case) needs no selection
        const int tok0 = t0p + 8 * vo;
        float sf[8], zf[8];
        halves_to_f32(s.vs, sf);
        halves_to_f32(s.vz, zf);
        uint4 vals[CPT];
        if (t0p + VPAGE <= vq && s.page >= 0) {
#pragma unroll
            for (int k = 0; k < CPT; ++k) vals[k] = dequant8<BITS>(s.vw[k], BITS == 4 ? 0 : (vo & 1), sf, zf);
        } else {
            const uint32_t below_vq = vq - tok0 >= 8 ? 0xFFu : (vq > tok0 ? (1u << (vq - tok0)) - 1u : 0u);
            const uint32_t from_codes = s.page >= 0 ? below_vq : 0u;
            const int end = min(row_len - tok0, 8);
            const uint32_t below_end = end >= 8 ? 0xFFu : (end > 0 ? (1u << end) - 1u : 0u);
            const uint32_t from_ring = below_end & ~below_vq;
#pragma unroll
            for (int k = 0; k < CPT; ++k)
                vals[k] = select8(from_codes, dequant8<BITS>(s.vw[k], BITS == 4 ? 0 : (vo & 1), sf, zf),
                                  make_uint4(0, 0, 0, 0));
            if (__ballot(from_ring != 0u) != 0) {  // the ring's tokens (the rows' last pages only)
#pragma unroll
                for (int k = 0; k < CPT; ++k) {
                    const int c = CPT * cq + k;
                    const uint4 x =
                        *reinterpret_cast<const uint4*>(p.v_ring + (row_kv * D + c) * p.ring + tok0 % p.ring);
                    vals[k] = select8(from_ring, x, vals[k]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < CPT; ++k)
            *reinterpret_cast<uint4*>(vl[buf] + (CPT * cq + k) * VROW + (VPAGE * pg + 8 * vo) * 2) = vals[k];
    };

    // ---- one tile of the wave's query rows from LDS buffer buf ----
    auto compute = [&](const Cursor& c, int buf, bool page0, bool page1) __attribute__((always_inline)) {
        const int t0 = VTILE * c.t;
        // S^T = K Q^T: block (kk, v) row m is token 32 kk + 8 (m / 4) + 4 v + m % 4, so lane (n, g) ends with tokens
        // 32 kk + 8 g + 4 v + i of query row r, the B operand of P.V
        f32x4 s[2][2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                s[kk][v] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                const uint8_t* krow = kl[buf] + (32 * kk + 8 * (n >> 2) + 4 * v + (n & 3)) * KROW + g * (D / 4) * 2;
#pragma unroll
                for (int j = 0; j < KS; ++j)
                    s[kk][v] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(krow + 16 * j)), qreg[j], s[kk][v],
                        0, 0, 0);
            }
        // the soft cap tested once per tile, not per score (the compiler keeps a uniform test inside an unrolled loop)
        if (p.softcap > 0.0f) {
            const float inv_cap = 1.0f / p.softcap;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int v = 0; v < 2; ++v)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        s[kk][v][i] = soft_cap_log2(s[kk][v][i] * score_scale, p.softcap, inv_cap);
        } else {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int v = 0; v < 2; ++v)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[kk][v][i] *= score_scale;
        }
        // masking where the tile holds a row's end, a causal limit, a missing codes page or a mask
        const bool missing = (!page0 && t0 < kq) || (!page1 && t0 + VPAGE < kq);
        if (t0 + VTILE > all_see || missing || p.mask) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const bool codes_ok = (kk == 0 ? page0 : page1) || t0 + VPAGE * kk >= kq;
                uint32_t word = 0xFFFFFFFFu;
                if (p.mask) word = mask_word(p, c.b, c.kvh, r, VerifyParams::kTile * c.t + kk);
#pragma unroll
                for (int v = 0; v < 2; ++v)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int e = 8 * g + 4 * v + i;
                        const bool ok = static_cast<float>(t0 + 32 * kk + e) < limit && codes_ok && ((word >> e) & 1u);
                        s[kk][v][i] = ok ? s[kk][v][i] : -INFINITY;
                    }
            }
        }
        // online softmax with lazy rescaling (the reference maximum moves when a score exceeds it by 2^8); the sum
        // stays lane-local until the segment ends
        float tile_max = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int v = 0; v < 2; ++v)
                tile_max = max_nan(max_nan(tile_max, max_nan(s[kk][v][0], s[kk][v][1])),
                                   max_nan(s[kk][v][2], s[kk][v][3]));
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
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            bf16x8 phi, plo;
#pragma unroll
            for (int v = 0; v < 2; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pw = __builtin_amdgcn_exp2f(s[kk][v][i] + neg_m);
                    l_i += pw;
                    phi[4 * v + i] = static_cast<__bf16>(pw);
                    plo[4 * v + i] = static_cast<__bf16>(pw - static_cast<float>(phi[4 * v + i]));
                }
            // O^T += V^T P^T: lane (n, g) supplies channel 16 nd + n of tokens 32 kk + 8 g .. 32 kk + 8 g + 7
#pragma unroll
            for (int nd = 0; nd < ND; ++nd) {
                const bf16x8 a = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const uint4*>(vl[buf] + (16 * nd + n) * VROW + (32 * kk + 8 * g) * 2));
                acc[nd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, phi, acc[nd], 0, 0, 0);
                acc[nd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, plo, acc[nd], 0, 0, 0);
            }
        }
    };

    // ---- end of a row segment: a whole row's output directly, else the segment's partial (max, sum, accumulators
    // of every query row) into the workgroup's slot for kivi_verify_merge_kernel ----
    auto finish = [&](const Cursor& c, int64_t seg_begin, int64_t seg_end, bool first_segment) __attribute__((always_inline)) {
        const float l = group_sum(l_i);
        if (seg_begin == c.row_start && seg_end == c.row_start + c.row.tiles) {
            if (r < p.rows)
#pragma unroll
                for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                    for (int i = 0; i < 4; ++i) store_output(p, c.b, c.kvh, r, 16 * nd + 4 * g + i, acc[nd][i], m_i, l);
            return;
        }
        // slot layout: accumulators [rows][D] first (8-byte aligned runs), then the maxima and the sums [rows]
        float* slot = p.part + (2 * static_cast<int64_t>(w) + (first_segment ? 0 : 1)) * p.rows * (D + 2);
        if (r < p.rows) {
            if (g == 0) {
                slot[p.rows * D + r] = m_i;
                slot[p.rows * D + p.rows + r] = l;
            }
#pragma unroll
            for (int nd = 0; nd < ND; ++nd) {
                float2* run = reinterpret_cast<float2*>(slot + r * D + 16 * nd + 4 * g);
                run[0] = make_float2(acc[nd][0], acc[nd][1]);
                run[1] = make_float2(acc[nd][2], acc[nd][3]);
            }
        }
    };

    // ---- the tile pipeline: tile pos is staged into LDS, then the next tile's loads are issued (past the range's
    // end a repeat of its last tile, read from L2 and never computed), then tile pos is computed ----
    Cursor cur = small ? locate_in(p, rt, lo) : locate(p, lo, lane);
    begin_row(cur);
    Cursor icur = cur;  // the tile the registers hold
    Share<D> sh;
    issue(sh, icur);
    int64_t seg_begin = lo;
    bool first_segment = true;
    for (int64_t pos = lo; pos < hi; ++pos) {
        cur = icur;
        if (cur.t == 0 && pos != lo) begin_row(cur);
        const int buf = static_cast<int>(pos & 1);
        const bool page0 = __builtin_amdgcn_readlane(win.physical, VerifyParams::kTile * cur.t - win.base) >= 0;
        const bool page1 = __builtin_amdgcn_readlane(win.physical, VerifyParams::kTile * cur.t + 1 - win.base) >= 0;
        stage(sh, cur, buf);
        if (pos + 1 < hi) advance(p, icur, small ? &rt : nullptr);
        issue(sh, icur);
        __syncthreads();
        compute(cur, buf, page0, page1);
        if (cur.t + 1 == cur.row.tiles || pos + 1 == hi) {
            finish(cur, seg_begin, pos + 1, first_segment);
            first_segment = false;
            seg_begin = pos + 1;
        }
    }
}

// The rows cut between workgroups, merged after the attention kernel (a second launch on the same stream, so the
// partials need no hand-off inside the first): one workgroup per (row, KV head) and 2048 of its rows x D outputs
// (blockIdx.y), so that a workgroup's loads are one round trip; a row whose tiles lie in one workgroup's range was
// written directly and is skipped. The parts are the workgroups whose ranges meet the row (slot
// 1 of a workgroup whose range starts before the row, else slot 0), folded by log-sum-exp four at a time, lane-owned
// runs of 8 channels of one query row, with the sinks in the denominator (attention/_decode_kernels.py:183-226).
template <int D>
__global__ __launch_bounds__(256) void kivi_verify_merge_kernel(VerifyParams p) {
    const int b = blockIdx.x / p.kv_heads, kvh = blockIdx.x % p.kv_heads;
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63;
    // the row's place in the tile sequence: rows before b (every KV head), then the KV heads before kvh
    int64_t before = 0;
    for (int b0 = 0; b0 < b; b0 += 64) {
        const int bb = b0 + lane;
        before += wave_sum(bb < b ? row_of(p, bb).tiles : 0);
    }
    int64_t total = before;
    for (int b0 = b; b0 < p.batch; b0 += 64) {
        const int bb = b0 + lane;
        total += wave_sum(bb < p.batch ? row_of(p, bb).tiles : 0);
    }
    total = uniform64(total * p.kv_heads);
    const int tiles = row_of<true>(p, b).tiles;
    if (tiles == 0) return;
    const int64_t row_start = uniform64(before * p.kv_heads + static_cast<int64_t>(kvh) * tiles);
    const int grid = p.grid;
    // the 64-bit divisions below are the same in every lane: done once per wave on uniform values
    const int w_first = uniform(wave_of(row_start, total, grid));
    const int w_last = uniform(wave_of(row_start + tiles - 1, total, grid));
    if (w_first == w_last) return;  // written directly
    const int64_t stride = static_cast<int64_t>(p.rows) * (D + 2);
    const int e = (static_cast<int>(blockIdx.y) * 256 + tid) * 8;
    if (e >= p.rows * D) return;
    const int rr = e / D, d = e % D;
    float m_run = -INFINITY, l_run = 0.0f, o_run[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o_run[i] = 0.0f;
    int64_t start_k = uniform64(total * w_first / grid);  // the first tile of workgroup k's range
    for (int k0 = w_first; k0 <= w_last; k0 += 4) {
        float mk[4], lk[4], ok[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int k = k0 + u;
            const int64_t end_k = uniform64(total * (k + 1) / grid);
            const bool use = k <= w_last && start_k < end_k;  // workgroup k holds a part of the row
            const float* sk = p.part + (2 * static_cast<int64_t>(use ? k : w_first) +
                                        (use && start_k < row_start ? 1 : 0)) * stride;
            mk[u] = use ? sk[p.rows * D + rr] : -INFINITY;
            lk[u] = use ? sk[p.rows * D + p.rows + rr] : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float2 x = use ? *reinterpret_cast<const float2*>(sk + rr * D + d + i) : make_float2(0.0f, 0.0f);
                ok[u][i] = x.x;
                ok[u][i + 1] = x.y;
            }
            start_k = end_k;
        }
        float m_new = m_run;
#pragma unroll
        for (int u = 0; u < 4; ++u) m_new = fmaxf(m_new, mk[u]);
        if (m_new == -INFINITY) continue;
        const float a = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= a;
#pragma unroll
        for (int i = 0; i < 8; ++i) o_run[i] *= a;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (mk[u] == -INFINITY) continue;
            const float cw = __builtin_amdgcn_exp2f(mk[u] - m_new);
            l_run += lk[u] * cw;
#pragma unroll
            for (int i = 0; i < 8; ++i) o_run[i] += ok[u][i] * cw;
        }
        m_run = m_new;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) store_output(p, b, kvh, rr, d + i, o_run[i], m_run, l_run);
}

template <typename F>
int verify_dispatch(int head_dim, int bits, const F& f) {
    if (head_dim == 64 && bits == 2) return f.template run<64, 2>();
    if (head_dim == 64 && bits == 4) return f.template run<64, 4>();
    if (head_dim == 128 && bits == 2) return f.template run<128, 2>();
    if (head_dim == 128 && bits == 4) return f.template run<128, 4>();
    return fail("kivi verification attention supports head dims 64 and 128 with 2- or 4-bit codes");
}

struct VerifyLaunch {
    hipStream_t stream;
    const KiviParams* p;
    template <int D, int BITS>
    int run() const {
        VerifyParams vp;
        static_cast<KiviParams&>(vp) = *p;
        hipLaunchKernelGGL((kivi_verify_kernel<D, BITS>), dim3(p->grid), dim3(256), 0, stream, vp);
        if (const int rc = check_launch("kivi_verify_kernel")) return rc;
        hipLaunchKernelGGL((kivi_verify_merge_kernel<D>), dim3(p->batch * p->kv_heads, (p->rows * D + 2047) / 2048),
                           dim3(256), 0, stream, vp);
        return check_launch("kivi_verify_merge_kernel");
    }
};

struct VerifyOccupancy {
    int* per_cu;
    template <int D, int BITS>
    int run() const {
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kivi_verify_kernel<D, BITS>, 256, 0) != hipSuccess ||
            blocks <= 0)
            blocks = 1;
        *per_cu = blocks;
        return 0;
    }
};

}  // namespace

int kivi_verify_resident_groups(int head_dim, int bits, int* per_cu) {
    return verify_dispatch(head_dim, bits, VerifyOccupancy{per_cu});
}

int kivi_verify_attention(const KiviParams& p, hipStream_t stream) {
    return verify_dispatch(p.head_dim, p.bits, VerifyLaunch{stream, &p});
}

}  // namespace eco
