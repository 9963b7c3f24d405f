// Split-K decode attention over a paged fp8 / bf16 KV cache on CDNA4 matrix cores (gfx950).
//
// What it computes is the reference's decode attention (attention/decode.py:66-103 as the definition,
// attention/_decode_kernels.py:110-226 for the split-K structure, log2-unit online softmax and the split merge):
// for every batch row b, KV head kvh and query row r = g * Q + qi of its group (query head h = kvh * G + g),
//   out[b, qi, h] = sum_t softmax_t(q . k_t * scale) v_t   over the row's visible tokens,
// with K/V decoded exactly from fp8 and multiplied by per-head scales. A page list turns it into Quest's gathered
// attention (attention/_quest_kernels.py:13-97): the virtual key axis is the selected pages, then the dense tail.
//
// Cache layout (vLLM's paged-attention layout, 16-token pages):
//   keys   [pages, Hkv, D / X, 16, X]  (X = 16 bytes of channels: 16 fp8 or 8 bf16)
//   values [pages, Hkv, D, 16]         (a channel's 16 tokens contiguous)
//
// Work decomposition. A workgroup handles one (split, kvh, b); its waves take tiles of 4 pages (64 tokens) in turn.
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
// O with the softmax weights P in fp16 (11 significant bits against the reference's bf16 rounding of P, which alone
// moves short rows by ~2^-9 of |v|). A bf16 cache multiplies its bf16 values by P split into two bf16 terms
// (P = P_hi + P_lo, 16 significant bits), two MFMAs per block.
//
// The waves of a workgroup merge their (max, sum, acc) in LDS. A row with one split writes its bf16 output directly;
// otherwise each split writes a partial and the last split of the row to finish (a per-(b, kvh) counter in the
// workspace) merges them by log-sum-exp (attention/_decode_kernels.py:183-226), so one launch does the whole call.

#include "common.hpp"
#include "paged_attention.hpp"

namespace eco {

namespace {

constexpr int PAGE = 16;

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

__device__ inline uint4 load16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

// First channel of k-step j (8 channels) for lane group g: run 4u + g of E channels, half h of it.
template <int E>
__device__ constexpr int k_channel(int j, int g) {
    constexpr int per_run = E / 8;
    return E * (4 * (j / per_run) + g) + 8 * (j % per_run);
}

// Logical page of virtual page v of row b (see paged_attention.hpp), -1 when it holds nothing.
__device__ inline int logical_page(const PagedParams& p, int b, int kvh, int v, int v_end, int done) {
    if (v >= v_end) return -1;
    int page = v;
    if (p.page_list != nullptr) page = v < p.n_sel ? p.page_list[b * p.pl_b + kvh * p.pl_h + v] : done + (v - p.n_sel);
    return page >= 0 && page < p.bt_cols ? page : -1;
}

}  // namespace

__device__ inline int virtual_pages(const PagedParams& p, int b, int* done_out) {
    const int len = p.seq_lens[b];
    const int pages = (len + PAGE - 1) / PAGE;
    if (p.page_list == nullptr) {
        *done_out = 0;
        return pages;
    }
    const int done = p.done[b];
    *done_out = done;
    return p.n_sel + max(0, pages - done);
}

// Splits that hold pages of a row with n_virt virtual pages (rows longer than the launch's max_seq_len are cut at
// the planned splits: their later pages are not read).
__device__ inline int row_splits(const PagedParams& p, int n_virt) {
    return n_virt <= 0 ? 0 : min((n_virt + p.split_pages - 1) / p.split_pages, p.max_splits);
}

// out[b, qi, h, d] of query row r from its merged (acc, max, sum) in log2 units, with the sink logit of head h in
// the denominator (attention/_decode_kernels.py:216-226): zeros for a row that sees nothing.
__device__ inline void store_output(const PagedParams& p, int b, int kvh, int r, int d, float o, float m, float l) {
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
    p.out[b * p.so_b + qi * p.so_q + h * p.so_h + d] = f32_to_bf16(out);
}

// Device-coherent (agent-scope) store and load of partials: they bypass the caches that are not coherent across the
// chip's XCDs (gfx950 lowers them to global_store / global_load with sc1), so no L2 writeback or invalidation is
// needed to hand a partial from one workgroup to another.
__device__ inline void coherent_store(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

__device__ inline float coherent_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Log-sum-exp merge of a row's split partials, in split order (attention/_decode_kernels.py:183-215).
template <int D>
__device__ inline void merge_splits(const PagedParams& p, int b, int kvh, int n_splits, int tid, int threads) {
    const int64_t part = (static_cast<int64_t>(b) * p.kv_heads + kvh) * p.max_splits * p.rows;
    for (int idx = tid; idx < p.rows * D; idx += threads) {
        const int r = idx / D;
        const int d = idx % D;
        float m = -INFINITY;
        for (int s = 0; s < n_splits; ++s) m = fmaxf(m, coherent_load(p.part_m + part + s * p.rows + r));
        float o = 0.0f, l = 0.0f;
        if (m != -INFINITY) {
            for (int s = 0; s < n_splits; ++s) {
                const float ms = coherent_load(p.part_m + part + s * p.rows + r);
                if (ms == -INFINITY) continue;
                const float c = __builtin_amdgcn_exp2f(ms - m);
                o += coherent_load(p.part_o + (part + s * p.rows + r) * D + d) * c;
                l += coherent_load(p.part_l + part + s * p.rows + r) * c;
            }
        }
        store_output(p, b, kvh, r, d, o, m, l);
    }
}

template <int D, int FMT, int NB, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void paged_split_kernel(PagedParams p) {
    constexpr int ES = FMT == BF16 ? 2 : 1;  // bytes per element
    constexpr int E = 16 / ES;               // channels per 16-byte run
    constexpr int NU = D * ES / 64;          // 16-byte K loads per lane per S MFMA block
    constexpr int KS = D / 32;               // k-steps of an S MFMA block
    constexpr int ND = D / 16;               // value blocks of 16 channels
    constexpr int NV = ES;                   // 16-byte V loads per lane per value block
    constexpr int KPR = E / 8;               // k-steps per run

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;

    int done = 0;
    const int n_virt = virtual_pages(p, b, &done);
    const int v_begin = split * p.split_pages;
    if (v_begin >= n_virt) {  // uniform over the workgroup: this split of the row is empty
        if (p.fused && split == 0) {  // a row with no key: zeros (sinks included, decode.py:17)
            for (int idx = threadIdx.x; idx < p.rows * D; idx += 64 * WAVES)
                store_output(p, b, kvh, idx / D, idx % D, 0.0f, -INFINITY, 0.0f);
        }
        return;
    }
    const int v_end = min(v_begin + p.split_pages, n_virt);
    const int len = p.seq_lens[b];

    // ---- query operand (B of the S MFMAs): column n = query row nb * 16 + n ----
    bf16x8 qop[NB][KS];
    float limit[NB];  // tokens at positions < limit are visible to the column
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int r = nb * 16 + n;
        const bool valid = r < p.rows;
        const int gq = valid ? r / p.queries : 0;
        const int qi = valid ? r % p.queries : 0;
        const int h = kvh * p.groups + gq;
        const uint16_t* base = p.q + b * p.sq_b + qi * p.sq_q + h * p.sq_h;
        limit[nb] = valid ? static_cast<float>(len - p.queries + qi + 1) : 0.0f;
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            uint4 raw = valid ? *reinterpret_cast<const uint4*>(base + k_channel<E>(j, g)) : make_uint4(0, 0, 0, 0);
            qop[nb][j] = __builtin_bit_cast(bf16x8, raw);
        }
    }
    const float ks = p.k_scale ? p.k_scale[kvh] : 1.0f;
    const float vs = p.v_scale ? p.v_scale[kvh] : 1.0f;
    const float score_scale = p.softcap > 0.0f ? p.scale * ks : p.scale * ks * kLog2e;

    const uint8_t* kbase = p.k_cache + kvh * p.kc_head;
    const uint8_t* vbase = p.v_cache + kvh * p.vc_head;
    const int32_t* table = p.block_table + b * p.bt_stride;

    float m_i[NB], l_i[NB];
    f32x4 acc[ND][NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        m_i[nb] = -INFINITY;
        l_i[nb] = 0.0f;
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) acc[nd][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    for (int t0 = v_begin + 4 * wave; t0 < v_end; t0 += 4 * WAVES) {
        // pages: the K rows of lane (n, g) come from tile page n / 4, its V channel from tile page g
        const int lk = logical_page(p, b, kvh, t0 + (n >> 2), v_end, done);
        const int lv = logical_page(p, b, kvh, t0 + g, v_end, done);
        int pk = lk >= 0 ? table[lk] : -1;
        int pv = lv >= 0 ? table[lv] : -1;
        pk = pk < p.num_pages ? pk : -1;  // a table entry outside the cache reads nothing
        pv = pv < p.num_pages ? pv : -1;

        uint4 kraw[4][NU];
        uint4 vraw[ND][NV];
        if (pk >= 0) {
            const uint8_t* kp = kbase + static_cast<int64_t>(pk) * p.kc_page;
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int u = 0; u < NU; ++u) kraw[v][u] = load16(kp + ((4 * u + g) * PAGE + 4 * v + (n & 3)) * 16);
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int u = 0; u < NU; ++u) kraw[v][u] = make_uint4(0, 0, 0, 0);
        }
        if (pv >= 0) {
            const uint8_t* vp = vbase + static_cast<int64_t>(pv) * p.vc_page;
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                for (int w = 0; w < NV; ++w) vraw[nd][w] = load16(vp + (16 * nd + n) * PAGE * ES + 16 * w);
        } else {
#pragma unroll
            for (int nd = 0; nd < ND; ++nd)
#pragma unroll
                for (int w = 0; w < NV; ++w) vraw[nd][w] = make_uint4(0, 0, 0, 0);
        }

        // ---- S^T = K Q^T: s[v][nb][i] = score of column n against token 4v + i of tile page g ----
        f32x4 s[4][NB];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s[v][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const uint4 run = kraw[v][j / KPR];
                bf16x8 a;
                if constexpr (FMT == BF16) {
                    a = __builtin_bit_cast(bf16x8, run);
                } else {
                    const int h2 = j % KPR;
                    a = fp8x8_to_bf16x8<FMT>(h2 ? run.z : run.x, h2 ? run.w : run.y);
                }
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    s[v][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qop[nb][j], s[v][nb], 0, 0, 0);
            }
        }

        // ---- online softmax per column, P^T operands ----
        // P operands: fp16 for fp8 caches, bf16 hi + lo for bf16 caches
        f16x8 pop_h[NB][2];
        bf16x8 pop_hi[NB][2], pop_lo[NB][2];
        const int first = lv * PAGE;  // position of token 0 of tile page g (lv < 0: nothing)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            float tile_max = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int pos = first + 4 * v + i;
                    const bool ok = lv >= 0 && static_cast<float>(pos) < limit[nb];
                    float x = s[v][nb][i] * score_scale;
                    if (p.softcap > 0.0f) {
                        const float t = x / p.softcap;
                        const float e = __expf(-2.0f * fabsf(t));
                        const float th = (1.0f - e) / (1.0f + e);
                        x = p.softcap * (t < 0.0f ? -th : th) * kLog2e;
                    }
                    x = ok ? x : -INFINITY;
                    s[v][nb][i] = x;
                    tile_max = fmaxf(tile_max, x);
                }
            tile_max = group_max(tile_max);
            const float m_new = fmaxf(m_i[nb], tile_max);
            const float m_safe = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_i[nb] - m_safe);
            float sum = 0.0f;
            float pv_[4][4];
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pv_[v][i] = __builtin_amdgcn_exp2f(s[v][nb][i] - m_safe);
                    sum += pv_[v][i];
                }
            sum = group_sum(sum);
            l_i[nb] = l_i[nb] * alpha + sum;
            m_i[nb] = m_new;
#pragma unroll
            for (int nd = 0; nd < ND; ++nd) acc[nd][nb] *= alpha;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float* a = pv_[2 * u];
                const float* c = pv_[2 * u + 1];
                if constexpr (FMT == BF16) {
                    float lo[8];
                    uint4 w;
                    w.x = pack_bf16x2(a[0], a[1]);
                    w.y = pack_bf16x2(a[2], a[3]);
                    w.z = pack_bf16x2(c[0], c[1]);
                    w.w = pack_bf16x2(c[2], c[3]);
                    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
                    const float vals[8] = {a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        lo[e] = vals[e] - bits_f32((e & 1 ? words[e >> 1] & 0xFFFF0000u : words[e >> 1] << 16));
                    uint4 z;
                    z.x = pack_bf16x2(lo[0], lo[1]);
                    z.y = pack_bf16x2(lo[2], lo[3]);
                    z.z = pack_bf16x2(lo[4], lo[5]);
                    z.w = pack_bf16x2(lo[6], lo[7]);
                    pop_hi[nb][u] = __builtin_bit_cast(bf16x8, w);
                    pop_lo[nb][u] = __builtin_bit_cast(bf16x8, z);
                } else {
                    uint4 w;
                    w.x = pack_f16x2(a[0], a[1]);
                    w.y = pack_f16x2(a[2], a[3]);
                    w.z = pack_f16x2(c[0], c[1]);
                    w.w = pack_f16x2(c[2], c[3]);
                    pop_h[nb][u] = __builtin_bit_cast(f16x8, w);
                }
            }
        }

        // ---- O^T += V^T P^T: lane (n, g) supplies channel 16 nd + n of tile page g ----
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if constexpr (FMT == BF16) {
                    const bf16x8 a = __builtin_bit_cast(bf16x8, vraw[nd][u]);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pop_hi[nb][u], acc[nd][nb], 0, 0, 0);
                        acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pop_lo[nb][u], acc[nd][nb], 0, 0, 0);
                    }
                } else {
                    const uint4 run = vraw[nd][0];
                    const f16x8 a = fp8x8_to_f16x8<FMT>(u ? run.z : run.x, u ? run.w : run.y);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[nd][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pop_h[nb][u], acc[nd][nb], 0, 0, 0);
                }
            }
        }
    }

    // ---- merge the waves in LDS ----
    // acc fragment of lane (n, g): channel 16 nd + 4 g + i of column nb * 16 + n.
    constexpr int SLOTS = ND * NB * 4;
    __shared__ float lds_acc[WAVES][SLOTS][64];
    __shared__ float lds_m[WAVES][16 * NB];
    __shared__ float lds_l[WAVES][16 * NB];
    __shared__ int lds_last;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < 4; ++i) lds_acc[wave][(nd * NB + nb) * 4 + i][lane] = acc[nd][nb][i];
    if (g == 0) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            lds_m[wave][nb * 16 + n] = m_i[nb];
            lds_l[wave][nb * 16 + n] = l_i[nb];
        }
    }
    __syncthreads();

    // A row with one split writes its output here; otherwise every split writes a partial (max, sum, acc) and the
    // last split of the row to finish merges them (a device-scope counter per (b, kvh), reset by that split).
    const int n_splits = row_splits(p, n_virt);
    const int64_t bh = static_cast<int64_t>(b) * p.kv_heads + kvh;
    const int64_t part = (bh * p.max_splits + split) * p.rows;
    const bool direct = p.fused && n_splits == 1;
    for (int idx = threadIdx.x; idx < p.rows * D; idx += 64 * WAVES) {
        const int r = idx / D;
        const int d = idx % D;
        const int nb = r >> 4;
        const int col = r & 15;
        const int slot = ((d >> 4) * NB + nb) * 4 + (d & 3);
        const int src_lane = ((d & 15) >> 2) * 16 + col;
        float m = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) m = fmaxf(m, lds_m[w][r]);
        float o = 0.0f, l = 0.0f;
        if (m != -INFINITY) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float mw = lds_m[w][r];
                if (mw == -INFINITY) continue;
                const float c = __builtin_amdgcn_exp2f(mw - m);
                o += lds_acc[w][slot][src_lane] * c;
                l += lds_l[w][r] * c;
            }
        }
        o *= vs;
        if (direct) {
            store_output(p, b, kvh, r, d, o, m, l);
        } else {
            coherent_store(p.part_o + (part + r) * D + d, o);
            if (d == 0) {
                coherent_store(p.part_m + part + r, m);
                coherent_store(p.part_l + part + r, l);
            }
        }
    }
    if (!p.fused || direct) return;
    // The partial was written with device-coherent stores: every wave waits until its stores completed (vmcnt 0),
    // the barrier joins the waves, then one thread counts the split. The last split reads the partials back with
    // device-coherent loads.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        lds_last = __hip_atomic_fetch_add(p.counters + bh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   n_splits - 1;
    __syncthreads();
    if (!lds_last) return;
    merge_splits<D>(p, b, kvh, n_splits, threadIdx.x, 64 * WAVES);
    if (threadIdx.x == 0) __hip_atomic_store(p.counters + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- host side ----------------------------------------------------------------------------------------------

namespace {

template <int D, int FMT, int NB>
int launch_split(const PagedParams& p, hipStream_t stream) {
    // the wave merge keeps WAVES * D * NB * 64 bytes in LDS: at most 64 KiB
    constexpr int FIT = 1024 / (D * NB);
    constexpr int WAVES = FIT >= 4 ? 4 : (FIT >= 1 ? FIT : 1);
    dim3 grid(p.max_splits, p.kv_heads, p.batch);
    hipLaunchKernelGGL((paged_split_kernel<D, FMT, NB, WAVES>), grid, dim3(64 * WAVES), 0, stream, p);
    return check_launch("paged_split_kernel");
}

template <int D, int FMT>
int dispatch_nb(const PagedParams& p, hipStream_t stream) {
    const int nb = (p.rows + 15) / 16;
    if (nb == 1) return launch_split<D, FMT, 1>(p, stream);
    if (nb == 2) return launch_split<D, FMT, 2>(p, stream);
    if (nb <= 4) return launch_split<D, FMT, 4>(p, stream);
    return fail("paged decode attention takes at most 64 query rows per KV head (query heads per KV head x queries)");
}

template <int D>
int dispatch_fmt(const PagedParams& p, hipStream_t stream) {
    switch (p.kv_format) {
        case BF16: return dispatch_nb<D, BF16>(p, stream);
        case FP8_E4M3: return dispatch_nb<D, FP8_E4M3>(p, stream);
        case FP8_E5M2: return dispatch_nb<D, FP8_E5M2>(p, stream);
        default: return fail("paged decode attention: KV format must be bf16, fp8 e4m3 or fp8 e5m2");
    }
}

}  // namespace

int paged_split(const PagedParams& p, hipStream_t stream) {
    switch (p.head_dim) {
        case 64: return dispatch_fmt<64>(p, stream);
        case 128: return dispatch_fmt<128>(p, stream);
        case 256: return dispatch_fmt<256>(p, stream);
        default: return fail("paged decode attention supports head dims 64, 128 and 256");
    }
}

}  // namespace eco
