// The stream-K machinery shared by the decode-attention kernels (paged_attention.hip, kivi.hip): the geometry of a
// row's tiles, the cursor over the sequence of every (row, KV head)'s tiles, the per-lane window of page ids, the
// output store with attention sinks, and the merge of the partials of a row cut between waves.
//
// A params type P provides: kPage (tokens per cache page), kTile (cache pages per tile), kPageList (whether it takes a
// Quest page list); the fields batch, kv_heads, rows, queries, groups, seq_lens, bt_cols, block_table, bt_stride,
// num_pages, sinks, out, so_b, so_q, so_h, counters, part, mask, mk_b, mk_h, mk_q, mask_words; and, with kPageList,
// page_list, pl_b, pl_h, n_sel, span, done.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace eco {
namespace {

__device__ inline int64_t wave_sum(int64_t x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

__device__ inline float wave_sum_f(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

__device__ inline float wave_max(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}

__device__ inline int64_t wave_inclusive_sum(int64_t x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    return x;
}

__device__ inline int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// The tile range of workgroup `block` of `grid`. Workgroups go to the 8 XCDs in turn (XCD block % 8); here each XCD
// takes a contiguous block of the ranges, so that neighbouring ranges (the same rows, the next KV heads) share an
// XCD's L2 and every XCD reads rows of every KV head. With range = block and one row per workgroup, XCD x read only
// KV head x of 8, a fixed 2 KB slot of every 16 KB page group: at the fp8 Llama-3-8B decode shape the even XCDs
// then finished their tiles 1.7 us before the odd ones.
__device__ inline int xcd_range(int block, int grid) {
    const int x = block & 7, k = block >> 3;
    const int q = grid >> 3, r = grid & 7;
    return x * q + min(x, r) + k;
}

// ptr[index] for a wave-uniform index through the scalar cache (a scalar load waits on its own counter, not on the
// vector loads in flight). Only for data no kernel of the call writes.
template <typename T>
__device__ inline T scalar_load(const T* ptr, int index) {
    return ((const __attribute__((address_space(4))) T*)ptr)[uniform(index)];
}

__device__ inline int64_t uniform64(int64_t x) {
    const uint64_t u = static_cast<uint64_t>(x);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// The optional attention mask, packed: bit t % 32 of word t / 32 of query row r of (b, kvh) says whether token t is
// visible (words [B][Hq][Q][mask_words] through the word strides mk_b, mk_h, mk_q, 0 on a broadcast axis). The word
// of tokens 32 w .. 32 w + 31; 0 (hidden) for a row past the group or a word past the mask.
template <typename P>
__device__ inline uint32_t mask_word(const P& p, int b, int kvh, int r, int w) {
    if (r >= p.rows || w < 0 || w >= p.mask_words) return 0u;
    const int gq = r / p.queries, qi = r % p.queries;
    return p.mask[b * p.mk_b + (kvh * p.groups + gq) * p.mk_h + qi * p.mk_q + w];
}

// Geometry of batch row b: tokens (cut at the block table's reach), where a page list's dense tail starts, and
// its virtual pages and tiles (the same for every KV head). UNIFORM: b is the same in every lane (scalar loads).
struct Row {
    int len, done, n_virt, tiles;
};

template <bool UNIFORM = false, typename P>
__device__ inline Row row_of(const P& p, int b) {
    Row r;
    const int len = UNIFORM ? scalar_load(p.seq_lens, b) : p.seq_lens[b];
    r.len = min(max(len, 0), p.bt_cols * P::kPage);
    const int pages = (r.len + P::kPage - 1) / P::kPage;
    r.done = 0;
    r.n_virt = pages;
    if constexpr (P::kPageList) {
        if (p.page_list != nullptr) {
            const int done = UNIFORM ? scalar_load(p.done, b) : p.done[b];
            r.done = min(max(done, 0) * p.span, pages);
            r.n_virt = p.n_sel * p.span + pages - r.done;
        }
    }
    r.tiles = (r.n_virt + P::kTile - 1) / P::kTile;
    return r;
}

// Logical page of virtual page v of a row, -1 when it holds nothing (past the row, an unselected list entry, or a
// listed page that is not committed).
template <typename P>
__device__ inline int logical_page(const P& p, const Row& row, int b, int kvh, int v) {
    if (v >= row.n_virt) return -1;
    if constexpr (P::kPageList) {
        if (p.page_list == nullptr) return v;
        const int listed = p.n_sel * p.span;
        if (v < listed) {
            const int entry = p.page_list[b * p.pl_b + kvh * p.pl_h + v / p.span];
            const int page = entry * p.span + v % p.span;
            return entry >= 0 && page < row.done ? page : -1;
        }
        return row.done + (v - listed);
    } else {
        return v;
    }
}

// Position in the tile sequence: row (b, kvh), its tile t, and the sequence offset of the row's first tile.
struct Cursor {
    int b, kvh, t;
    Row row;
    int64_t row_start;
};

template <typename P>
__device__ inline int64_t total_tiles(const P& p, int lane) {
    int64_t total = 0;
    for (int b0 = 0; b0 < p.batch; b0 += 64) {
        const int b = b0 + lane;
        total += wave_sum(b < p.batch ? row_of(p, b).tiles : 0);
    }
    return total * p.kv_heads;
}

// The cursor of sequence offset x < total_tiles.
template <typename P>
__device__ inline Cursor locate(const P& p, int64_t x, int lane) {
    Cursor c{};
    int64_t base = 0;
    for (int b0 = 0; b0 < p.batch; b0 += 64) {
        const int b = b0 + lane;
        const int tiles = b < p.batch ? row_of(p, b).tiles : 0;
        const int64_t incl = wave_inclusive_sum(static_cast<int64_t>(tiles) * p.kv_heads, lane);
        const int64_t chunk = __shfl(incl, 63);
        if (x < base + chunk) {
            const int src = __builtin_ctzll(__ballot(base + incl > x));
            c.b = uniform(b0 + src);
            c.row = row_of(p, c.b);
            c.row.len = uniform(c.row.len);
            c.row.done = uniform(c.row.done);
            c.row.n_virt = uniform(c.row.n_virt);
            c.row.tiles = uniform(c.row.tiles);
            const int64_t start_b =
                uniform64(base + __shfl(incl, src) - static_cast<int64_t>(c.row.tiles) * p.kv_heads);
            const int64_t off = x - start_b;
            c.kvh = uniform(static_cast<int>(off / c.row.tiles));
            c.t = uniform(static_cast<int>(off % c.row.tiles));
            c.row_start = uniform64(start_b + static_cast<int64_t>(c.kvh) * c.row.tiles);
            return c;
        }
        base += chunk;
    }
    return c;
}

// Batches of at most 64 rows: lane b holds row b's geometry and the inclusive sum of the tile counts (times the KV
// heads) up to it, from one load of the lengths; the total, the cursor of an offset and the next row then come from
// lane reads instead of loads.
struct RowTable {
    Row row;
    int64_t incl;
};

template <typename P>
__device__ inline RowTable row_table(const P& p, int lane) {
    RowTable t;
    t.row = lane < p.batch ? row_of(p, lane) : Row{0, 0, 0, 0};
    t.incl = wave_inclusive_sum(static_cast<int64_t>(t.row.tiles) * p.kv_heads, lane);
    return t;
}

__device__ inline Row row_at(const RowTable& t, int b) {
    Row r;
    r.len = __builtin_amdgcn_readlane(t.row.len, b);
    r.done = __builtin_amdgcn_readlane(t.row.done, b);
    r.n_virt = __builtin_amdgcn_readlane(t.row.n_virt, b);
    r.tiles = __builtin_amdgcn_readlane(t.row.tiles, b);
    return r;
}

// The cursor of sequence offset x < total, from the row table.
template <typename P>
__device__ inline Cursor locate_in(const P& p, const RowTable& t, int64_t x) {
    Cursor c{};
    const int b = uniform(__builtin_ctzll(__ballot(t.incl > x)));
    c.b = b;
    c.row = row_at(t, b);
    const int64_t start_b = uniform64(__shfl(t.incl, b)) - static_cast<int64_t>(c.row.tiles) * p.kv_heads;
    const int64_t off = x - start_b;
    c.kvh = uniform(static_cast<int>(off / c.row.tiles));
    c.t = uniform(static_cast<int>(off % c.row.tiles));
    c.row_start = uniform64(start_b + static_cast<int64_t>(c.kvh) * c.row.tiles);
    return c;
}

// The next tile (called only when one exists); rows come from the table when one is given.
template <typename P>
__device__ inline void advance(const P& p, Cursor& c, const RowTable* table = nullptr) {
    if (++c.t < c.row.tiles) return;
    c.row_start += c.row.tiles;
    c.t = 0;
    if (++c.kvh < p.kv_heads) return;
    c.kvh = 0;
    do {
        c.b = uniform(c.b + 1);
        if (table) {
            c.row = row_at(*table, c.b);
        } else {
            c.row = row_of<true>(p, c.b);
            c.row.len = uniform(c.row.len);
            c.row.done = uniform(c.row.done);
            c.row.n_virt = uniform(c.row.n_virt);
            c.row.tiles = uniform(c.row.tiles);
        }
    } while (c.row.tiles == 0 && c.b + 1 < p.batch);
}

// The tile at cursor position c.t of a row walked from its last tile down (position t is tile tiles - 1 - t): the
// cursor, the ranges and the merges count positions; the loads, token offsets and masks use the tile.
__device__ inline Cursor at_tile(const Cursor& c) {
    Cursor t = c;
    t.t = c.row.tiles - 1 - c.t;
    return t;
}

// The wave whose range holds sequence offset x.
__device__ inline int wave_of(int64_t x, int64_t total, int grid) {
    return static_cast<int>(((x + 1) * grid - 1) / total);
}

// The 16-bit output element of x: fp16 where the call's queries are fp16 (a parameter block with out_f16 set),
// else bf16.
template <typename P, typename = void>
struct HasOutF16 : std::false_type {};
template <typename P>
struct HasOutF16<P, std::void_t<decltype(P::out_f16)>> : std::true_type {};

template <typename P>
__device__ inline uint16_t out_bits(const P& p, float x) {
    if constexpr (HasOutF16<P>::value)
        if (p.out_f16) return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    return f32_to_bf16(x);
}

// out[b, qi, h, d] of query row r from its merged (acc, max, sum) in log2 units, with the sink logit of head h in
// the denominator (attention/_decode_kernels.py:216-226): zeros for a row that sees nothing.
template <typename P>
__device__ inline void store_output(const P& p, int b, int kvh, int r, int d, float o, float m, float l) {
    const int gq = r / p.queries;
    const int qi = r % p.queries;
    const int h = kvh * p.groups + gq;
    if (p.sinks) {
        const float sink = p.sinks[h] * kLog2e;
        const float m_new = fmaxf(m, sink);
        const float a = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - m_new);
        o *= a;
        l = l * a + __builtin_amdgcn_exp2f(sink - m_new);
    }
    const float out = l > 0.0f ? o / fmaxf(l, 1e-30f) : 0.0f;
    p.out[b * p.so_b + qi * p.so_q + h * p.so_h + d] = out_bits(p, out);
}

// Page ids of 64 consecutive virtual pages of one (b, kvh) row, one per lane: lane i holds the logical page and the
// cache page of virtual page base + i (-1 when it holds nothing). A tile's K/V addresses then come from a lane
// shuffle instead of a block-table load issued right before the K/V loads (whose latency the loads would wait out,
// and, since loads retire in order, with them every load in flight). The window is reloaded once per 16 tiles.
struct PageWindow {
    int b = -1, kvh = -1, base = 0;
    int logical = -1, physical = -1;
};

// DESCENDING: the row is walked from its last tile down, so a reload covers the 64 pages that end with the tile.
template <typename P, bool DESCENDING = false>
__device__ __forceinline__ void ensure_window(const P& p, const Cursor& c, int lane, PageWindow& win) {
    const int first = P::kTile * c.t;
    if (c.b == win.b && c.kvh == win.kvh && first >= win.base && first + P::kTile <= win.base + 64) return;
    win.b = c.b;
    win.kvh = c.kvh;
    win.base = DESCENDING ? max(first + P::kTile - 64, 0) : first;
    const int lp = logical_page(p, c.row, c.b, c.kvh, win.base + lane);
    int pp = lp >= 0 ? p.block_table[c.b * p.bt_stride + lp] : -1;
    pp = pp < p.num_pages ? pp : -1;  // a table entry outside the cache reads nothing
    win.logical = pp >= 0 ? lp : -1;
    win.physical = pp;
    // wait here for the table load (vmcnt(0)), so that the common path, which reloads nothing, does not wait at
    // the branch's join for every load in flight
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

// The hand-off of a row's partial, written by this wave with coherent_store, to the last of the row's parts. The
// partials are only ever written and read as agent-scope atomics (sc1: written through to, and read from, the level
// every XCD sees), so what orders the hand-off is completion, not cache maintenance: the compiler may not move the
// stores past the count (a signal fence), the wave waits until its stores are complete (vmcnt counts stores on
// gfx950), and only then lane 0 counts the part with an agent-scope atomic; the wave that finds every other part
// counted issues its loads after the atomic returned (merge_row, after a second signal fence). Agent-scope release /
// acquire fences (buffer_wbl2 / buffer_inv of the XCD's L2) would add nothing for sc1 data and cost 6 us on the
// ragged fp8 call and 10-12 us on the KIVI decode call, measured.
template <int D, typename P>
__device__ inline void merge_row(const P& p, const Cursor& c, int prev, int64_t total, int grid, int lane);

template <int D, typename P>
__device__ inline void hand_off(const P& p, const Cursor& c, int64_t total, int grid, int lane) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0), expcnt(0), lgkmcnt(0): every store of the partial is complete
    int prev = 0;
    if (lane == 0)
        prev = __hip_atomic_fetch_add(p.counters + c.b * p.kv_heads + c.kvh, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    merge_row<D>(p, c, __shfl(prev, 0), total, grid, lane);
}

// The merge of a row's partials by the last of its waves to finish: per query row, the maximum and the weighted sum
// over the partials (lanes over partials), then the weighted accumulators (lanes over channels). Returns without
// merging when other partials of the row are still outstanding.
template <int D, typename P>
__device__ inline void merge_row(const P& p, const Cursor& c, int prev, int64_t total, int grid,
                                       int lane) {
    const int64_t row_end = c.row_start + c.row.tiles;
    const int64_t stride = static_cast<int64_t>(p.rows) * (D + 2);
    int32_t* counter = p.counters + c.b * p.kv_heads + c.kvh;
        // the waves holding part of the row (a wave's range is empty only when there are fewer tiles than waves)
        const int w_first = wave_of(c.row_start, total, grid);
        const int w_last = wave_of(row_end - 1, total, grid);
        auto holds = [&](int k) __attribute__((always_inline)) { return total * k / grid < total * (k + 1) / grid; };
        auto slot_of = [&](int k) __attribute__((always_inline)) {
            return p.part + (2 * static_cast<int64_t>(k) + (total * k / grid < c.row_start ? 1 : 0)) * stride;
        };
        int parts = 0;
        for (int k = w_first + lane; k <= w_last; k += 64) parts += holds(k) ? 1 : 0;
        parts = static_cast<int>(wave_sum(parts));
        if (prev != parts - 1) return;
        // every other part's partial was complete before its count; the loads follow the count that found them
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // lane-owned runs of 8 channels of one query row; the partials are folded in batches of 4 with an online
        // log-sum-exp, the batch's loads all in flight together
        for (int base = 0; base < p.rows * D; base += 64 * 8) {
            const int e = base + lane * 8;
            const bool active = e < p.rows * D;
            const int r = active ? e / D : 0;
            const int d = active ? e % D : 0;
            float m_run = -INFINITY, l_run = 0.0f, o_run[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o_run[i] = 0.0f;
            for (int k0 = w_first; k0 <= w_last; k0 += 4) {
                float mk[4], lk[4], ok[4][8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = k0 + j;
                    const bool use = active && k <= w_last && holds(k);
                    const float* sk = slot_of(use ? k : w_first);
                    mk[j] = use ? coherent_load(sk + r) : -INFINITY;
                    lk[j] = use ? coherent_load(sk + p.rows + r) : 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) ok[j][i] = use ? coherent_load(sk + 2 * p.rows + r * D + d + i) : 0.0f;
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
            if (active)
#pragma unroll
                for (int i = 0; i < 8; ++i) store_output(p, c.b, c.kvh, r, d + i, o_run[i], m_run, l_run);
        }
        if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// ---- the pieces of rows inside one multi-wave workgroup ----------------------------------------------------------
// Each wave of a workgroup takes a contiguous part of the workgroup's tile range; its first and last row segments
// that are not whole rows are left in LDS as pieces (maxima, sums and output values of at most PR query rows). After
// a barrier the pieces are merged per row, the rows taken by the waves in turn: a row inside the workgroup's range is
// written out, a row cut at a range boundary becomes the workgroup's partial in the workspace (slot 0 when the row
// started before the workgroup, else slot 1) and joins the counter merge of merge_row. The two rows cut at the range's
// ends go to different waves, so that their workspace round trips (partial stores, counter, the last part's merge)
// overlap instead of following each other.
template <int D, int WAVES, int PR = 16>
struct Pieces {
    // a piece: the output values of `rows` query rows [r * D + d], then their maxima [rows * D + r], then their sums
    __align__(16) float data[2 * WAVES][PR * (D + 2)];
    int64_t row[2 * WAVES];  // row_start of the piece's row, -1 for none
    int b[2 * WAVES], kvh[2 * WAVES], tiles[2 * WAVES];
};

template <int D, int WAVES, int PR>
__device__ inline void clear_pieces(Pieces<D, WAVES, PR>& pc, int wave, int lane) {
    if (lane < 2) pc.row[2 * wave + lane] = -1;
}

// Stores the segment of row c as piece k: lane (n, g) holds query row n's output channels 16 nd + 4 g + i
// (value(nd, i)), and m, l of row n; four channels per 16-byte LDS store.
template <int D, int WAVES, int PR, typename V>
__device__ __forceinline__ void write_piece(Pieces<D, WAVES, PR>& pc, int k, const Cursor& c, int rows, int n, int g,
                                            int lane, float m, float l, V value) {
    float* piece = pc.data[k];
    if (n < rows) {
        if (g == 0) {
            piece[rows * D + n] = m;
            piece[rows * D + rows + n] = l;
        }
#pragma unroll
        for (int nd = 0; nd < D / 16; ++nd)
            *reinterpret_cast<float4*>(piece + n * D + 16 * nd + 4 * g) =
                make_float4(value(nd, 0), value(nd, 1), value(nd, 2), value(nd, 3));
    }
    if (lane == 0) {
        pc.row[k] = c.row_start;
        pc.b[k] = c.b;
        pc.kvh[k] = c.kvh;
        pc.tiles[k] = c.row.tiles;
    }
}

// out[b, qi, h, d .. d + 1] of query row r (d even) from its merged accumulators o0, o1, maximum m and sum l (log2
// units), with the sink logit of head h in the denominator: one 4-byte store where the address allows.
template <typename P>
__device__ inline void store_output2(const P& p, int b, int kvh, int r, int d, float o0, float o1, float m, float l) {
    const int gq = r / p.queries;
    const int qi = r % p.queries;
    const int h = kvh * p.groups + gq;
    if (p.sinks) {
        const float sink = p.sinks[h] * kLog2e;
        const float m_new = fmaxf(m, sink);
        const float a = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - m_new);
        o0 *= a;
        o1 *= a;
        l = l * a + __builtin_amdgcn_exp2f(sink - m_new);
    }
    const float inv = l > 0.0f ? 1.0f / fmaxf(l, 1e-30f) : 0.0f;
    uint16_t* out = p.out + b * p.so_b + qi * p.so_q + h * p.so_h + d;
    const uint32_t pair = static_cast<uint32_t>(out_bits(p, o0 * inv)) | (static_cast<uint32_t>(out_bits(p, o1 * inv)) << 16);
    if ((reinterpret_cast<uintptr_t>(out) & 3) == 0) {
        *reinterpret_cast<uint32_t*>(out) = pair;
    } else {
        out[0] = static_cast<uint16_t>(pair);
        out[1] = static_cast<uint16_t>(pair >> 16);
    }
}

template <int D, int WAVES, int PR, typename P>
__device__ inline void merge_pieces(const P& p, Pieces<D, WAVES, PR>& pc, int wave, int lane, int64_t wlo, int64_t whi,
                                    int64_t total, int grid, int w) {
    constexpr int K = 2 * WAVES;  // piece slots
    __syncthreads();
    const int64_t stride = static_cast<int64_t>(p.rows) * (D + 2);
    const int vals = p.rows * D;  // offset of a piece's maxima (its sums follow them)
    // The piece table in one read (lane j < K holds piece j), so that finding the rows and their pieces takes no
    // further LDS round trip: at the end of the call this merge is on the critical path of the workgroup.
    const bool holder = lane < K;
    int64_t prow = holder ? pc.row[lane] : -1;
    const int pb = holder ? pc.b[lane] : 0;
    const int pkvh = holder ? pc.kvh[lane] : 0;
    const int ptiles = holder ? pc.tiles[lane] : 0;
    int group = 0;
    for (;;) {
        const uint64_t live = __ballot(prow >= 0);
        if (live == 0) break;
        const int k = static_cast<int>(__builtin_ctzll(live));  // the first piece of the next row (pieces follow the tiles)
        const int64_t row = uniform64(__shfl(prow, k));
        const uint32_t members = static_cast<uint32_t>(__ballot(prow == row));
        if (prow == row) prow = -1;
        Cursor c{};
        c.b = uniform(__shfl(pb, k));
        c.kvh = uniform(__shfl(pkvh, k));
        c.row.tiles = uniform(__shfl(ptiles, k));
        c.row_start = row;
        const bool inside = row >= wlo && row + c.row.tiles <= whi;
        if (inside) {
            // a row inside the workgroup: every wave merges a share of its outputs, two channels per lane, and writes
            // them; every slot is read (the reads in flight together) and a slot outside the row weighs nothing
            for (int e = 2 * (wave * 64 + lane); e < vals; e += 2 * 64 * WAVES) {
                const int r = e / D, d = e % D;
                float mj[K], lj[K];
                float2 vj[K];
#pragma unroll
                for (int j = 0; j < K; ++j) {
                    mj[j] = pc.data[j][vals + r];
                    lj[j] = pc.data[j][vals + p.rows + r];
                    vj[j] = *reinterpret_cast<const float2*>(&pc.data[j][r * D + d]);
                }
                float m = -INFINITY;
#pragma unroll
                for (int j = 0; j < K; ++j)
                    if ((members >> j) & 1u) m = fmaxf(m, mj[j]);
                float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
                for (int j = 0; j < K; ++j) {
                    if (!((members >> j) & 1u) || mj[j] == -INFINITY) continue;
                    const float cw = __builtin_amdgcn_exp2f(mj[j] - m);
                    l += lj[j] * cw;
                    o0 += vj[j].x * cw;
                    o1 += vj[j].y * cw;
                }
                store_output2(p, c.b, c.kvh, r, d, o0, o1, m, l);
            }
            continue;
        }
        // a row cut at the workgroup's range: one wave writes the workgroup's partial and joins the row's merge
        if (group++ % WAVES != wave) continue;
        float* slot = p.part + (2 * static_cast<int64_t>(w) + (wlo < row ? 1 : 0)) * stride;
        for (int base = 0; base < vals; base += 64 * 8) {
            const int e = base + lane * 8;
            const bool active = e < vals;
            const int r = active ? e / D : 0;
            const int d = active ? e % D : 0;
            float mj[K];
#pragma unroll
            for (int j = 0; j < K; ++j) mj[j] = pc.data[j][vals + r];
            float m = -INFINITY;
#pragma unroll
            for (int j = 0; j < K; ++j)
                if ((members >> j) & 1u) m = fmaxf(m, mj[j]);
            float l = 0.0f, o[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < K; ++j) {
                if (!((members >> j) & 1u) || mj[j] == -INFINITY) continue;
                const float cw = __builtin_amdgcn_exp2f(mj[j] - m);
                l += pc.data[j][vals + p.rows + r] * cw;
                const float4 v0 = *reinterpret_cast<const float4*>(&pc.data[j][r * D + d]);
                const float4 v1 = *reinterpret_cast<const float4*>(&pc.data[j][r * D + d + 4]);
                o[0] += v0.x * cw;
                o[1] += v0.y * cw;
                o[2] += v0.z * cw;
                o[3] += v0.w * cw;
                o[4] += v1.x * cw;
                o[5] += v1.y * cw;
                o[6] += v1.z * cw;
                o[7] += v1.w * cw;
            }
            if (!active) continue;
            if (d == 0) {
                coherent_store(slot + r, m);
                coherent_store(slot + p.rows + r, l);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) coherent_store(slot + 2 * p.rows + r * D + d + i, o[i]);
        }
        // the workgroup's partial joins the others' in the workspace; the last workgroup to finish merges them
        hand_off<D>(p, c, total, grid, lane);
    }
}


}  // namespace
}  // namespace eco
