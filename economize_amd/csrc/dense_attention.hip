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
// (the lo.lo term is below fp32 rounding of the sum). The softmax weights p are split the same way for P.V.
//
// Work split (flash-decoding, as the reference): the key axis is cut into splits of split_len keys; one wave takes
// one (row, KV head, block of 16 query rows, split) and walks its split in tiles of 32 keys; a merge kernel combines
// the splits by log-sum-exp. Per tile, S^T = K Q^T with v_mfma_f32_16x16x32_bf16: A-row m of MFMA block v is key
// 8 (m / 4) + 4 v + m % 4, so that lane (n, g) ends with keys 8 g .. 8 g + 7 of query row n, which is exactly the B
// operand of O^T += V^T P^T; the keys are read token-major from HBM straight into the A operand (16-byte loads).
// V^T needs a lane to hold 8 keys of one channel: the tile's values are staged through LDS (coalesced 16-byte loads,
// rows padded by 16 bytes so that the four lane groups' reads fall in different banks) and read back transposed.

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

// The raw words of eight consecutive elements of format FMT at p (16-byte aligned; fp8: 8-byte aligned).
template <int FMT>
__device__ __forceinline__ void load8(const uint8_t* p, uint4 (&w)[FMT == FP32 ? 2 : 1]) {
    if constexpr (FMT == FP8_E4M3 || FMT == FP8_E5M2) {
        const uint2 x = *reinterpret_cast<const uint2*>(p);
        w[0] = make_uint4(x.x, x.y, 0, 0);
    } else {
#pragma unroll
        for (int i = 0; i < (FMT == FP32 ? 2 : 1); ++i) w[i] = reinterpret_cast<const uint4*>(p)[i];
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

template <int QF>
__device__ __forceinline__ void load_query8(const DenseParams& p, int64_t offset, bf16x8& hi, bf16x8& lo) {
    uint4 w[QF == FP32 ? 2 : 1];
    load8<QF>(static_cast<const uint8_t*>(p.q) + offset * elem_bytes<QF>(), w);
    cvt8<QF>(w, hi, lo);
}

template <int DP, int FMT, int QF>
__global__ __launch_bounds__(64) void dense_split_kernel(DenseParams p) {
    constexpr int ES = elem_bytes<FMT>();
    constexpr int KS = DP / 32;  // k-steps of the S MFMA
    constexpr int ND = DP / 16;  // value blocks of 16 channels
    constexpr bool KLO = two_terms<FMT>();
    constexpr bool QLO = two_terms<QF>();
    constexpr int ROW = DP * ES + 16;  // LDS bytes per staged value row
    __shared__ __align__(16) uint8_t vtile[TK * ROW];

    const int lane = static_cast<int>(threadIdx.x);
    const int n = lane & 15, g = lane >> 4;
    const int prog = blockIdx.x;
    const int split = blockIdx.y;
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
        if (r_ok && c < p.head_dim)
            load_query8<QF>(p, b * p.sq_b + h * p.sq_h + static_cast<int64_t>(q_start + qi) * p.sq_q + c, qh[j], ql[j]);
    }
    const float ks = p.k_scale ? p.k_scale[kvh] : 1.0f;
    const float vs = p.v_scale ? p.v_scale[kvh] : 1.0f;
    const float score_scale = p.softcap > 0.0f ? p.scale * ks : p.scale * ks * kLog2e;
    const float inv_cap = p.softcap > 0.0f ? 1.0f / p.softcap : 0.0f;
    const uint8_t* kbase = static_cast<const uint8_t*>(p.k) + (b * p.sk_b + kvh * p.sk_h) * ES;
    const uint8_t* vbase = static_cast<const uint8_t*>(p.v) + (b * p.sv_b + kvh * p.sv_h) * ES;
    const uint8_t* mrow = p.mask ? p.mask + b * p.sm_b + h * p.sm_h + qi * p.sm_q : nullptr;
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
    // cells: the cache pages of the current tile's two 16-key halves, looked up once per tile (tile_pages)
    int64_t cell_half[2] = {0, 0};
    auto page_base = [&](int t) __attribute__((always_inline)) -> int64_t {
        const int lp = min(t / p.page_size, p.bt_cols - 1);
        const int page = min(max(p.block_table[static_cast<int64_t>(b) * p.bt_stride + lp], 0), p.num_pages - 1);
        return page * p.sc_page + kvh * p.sc_head;
    };
    auto tile_pages = [&](int t0) __attribute__((always_inline)) {
        if (p.cells) {
            cell_half[0] = page_base(t0);
            cell_half[1] = p.page_size % 32 == 0 ? cell_half[0] : page_base(t0 + 16);
        }
    };
    auto cell_row = [&](int t) __attribute__((always_inline)) -> const uint8_t* {
        // a tile starts at a multiple of 32 keys and pages hold a multiple of 16, so each 16-key half lies in one page
        return p.cells + cell_half[(t >> 4) & 1] + static_cast<int64_t>(t % p.page_size) * p.sc_token;
    };
    auto key_row = [&](int t) __attribute__((always_inline)) -> const uint8_t* {
        if (p.cells) return cell_row(t);
        return t < count ? gkbase + static_cast<int64_t>(t) * p.sgk_s * ES
                         : kbase + static_cast<int64_t>(start + t - count) * p.sk_s * ES;
    };
    auto value_row = [&](int t) __attribute__((always_inline)) -> const uint8_t* {
        if (p.cells) return cell_row(t) + p.cell_off_v;
        return t < count ? gvbase + static_cast<int64_t>(t) * p.sgv_s * ES
                         : vbase + static_cast<int64_t>(start + t - count) * p.sv_s * ES;
    };
    // causal: the last q_count keys of the row are its queries' own tokens
    const int causal_limit = p.causal ? row_keys - q_count + qi + 1 : row_keys;
    auto mask_col = [&](int t) __attribute__((always_inline)) -> int64_t {
        return t < count ? min(max(gidx[t], 0), p.dense_keys - 1) : start + t - count;
    };

    float m_i = -INFINITY, l_i = 0.0f;
    f32x4 acc[ND];
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) acc[nd] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int t_begin = split * p.split_len;
    const int t_end = min(row_keys, t_begin + p.split_len);
    constexpr int CHUNKS = TK * DP * ES / 16;  // 16-byte chunks of a staged value tile
    constexpr int CPR = DP * ES / 16;          // chunks per value row
    constexpr int CPL = (CHUNKS + 63) / 64;    // chunks per lane
    constexpr bool kStage = CPL <= 8;          // the tile's values pass through registers (loads issued first)
    constexpr int KW = ES == 4 ? 2 : 1;        // 16-byte words of 8 key elements (fp8: the low half of one)
    for (int t0 = t_begin; t0 < t_end; t0 += TK) {
        tile_pages(t0);
        // ---- issue the tile's loads: values (staged for LDS), then keys (A-row n of block v is key
        // t0 + 8 (n / 4) + 4 v + n % 4; a key past the split reads the split's last key and is masked) ----
        auto value_chunk = [&](int chunk) __attribute__((always_inline)) -> uint4 {
            const int t = chunk / CPR;
            const int c = (chunk % CPR) * (16 / ES);  // first channel of the chunk
            if (chunk < CHUNKS && t0 + t < t_end && c < p.value_dim)
                return *reinterpret_cast<const uint4*>(value_row(t0 + t) + c * ES);
            return make_uint4(0, 0, 0, 0);
        };
        uint4 vreg[kStage ? CPL : 1];
        if constexpr (kStage)
#pragma unroll
            for (int i = 0; i < CPL; ++i) vreg[i] = value_chunk(lane + 64 * i);
        uint4 kr[2][KS][KW];
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int tk = min(t0 + 8 * (n >> 2) + 4 * v + (n & 3), t_end - 1);
            const uint8_t* krow = key_row(tk);
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const int c = 32 * j + 8 * g;
#pragma unroll
                for (int w = 0; w < KW; ++w) kr[v][j][w] = make_uint4(0, 0, 0, 0);
                if (c < p.head_dim) load8<FMT>(krow + c * ES, kr[v][j]);
            }
        }
        // ---- the values into LDS (zero past the keys and past Dv) ----
        if constexpr (kStage) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int chunk = lane + 64 * i;
                if (chunk < CHUNKS) *reinterpret_cast<uint4*>(vtile + (chunk / CPR) * ROW + (chunk % CPR) * 16) = vreg[i];
            }
        } else {
            for (int chunk = lane; chunk < CHUNKS; chunk += 64)
                *reinterpret_cast<uint4*>(vtile + (chunk / CPR) * ROW + (chunk % CPR) * 16) = value_chunk(chunk);
        }
        // ---- S^T = K Q^T ----
        f32x4 s[2];
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            s[v] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                bf16x8 kh, kl;
                cvt8<FMT>(kr[v][j], kh, kl);
                s[v] = mfma(kh, qh[j], s[v]);
                if constexpr (QLO) s[v] = mfma(kh, ql[j], s[v]);
                if constexpr (KLO) s[v] = mfma(kl, qh[j], s[v]);
            }
        }
        // ---- scores in log2 units, masked: lane (n, g) holds keys t0 + 8 g + 4 v + i of row r ----
        uint32_t vis = 0;  // bit 4 v + i
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int t = t0 + 8 * g + e;
            bool ok = r_ok && t < t_end && t < causal_limit;
            if (ok && mrow) ok = mrow[mask_col(t) * p.sm_s] != 0;
            vis |= ok ? 1u << e : 0u;
        }
        float tile_max = -INFINITY;
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = s[v][i] * score_scale;
                if (p.softcap > 0.0f) x = soft_cap_log2(x, p.softcap, inv_cap);
                x = (vis >> (4 * v + i)) & 1u ? x : -INFINITY;
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
        split8(pw, ph, pl);
        // ---- O^T += V^T P^T: lane (n, g) supplies channel 16 nd + n of keys 8 g .. 8 g + 7 ----
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tile's LDS stores (one wave: in order)
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) {
            const int c = 16 * nd + n;
            if (16 * nd >= p.value_dim) break;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = elem_f32<FMT>(vtile + (8 * g + e) * ROW + c * ES);
            bf16x8 vh, vl;
            split8(x, vh, vl);
            acc[nd] = mfma(vh, ph, acc[nd]);
            acc[nd] = mfma(vh, pl, acc[nd]);
            if constexpr (KLO) acc[nd] = mfma(vl, ph, acc[nd]);
        }
    }
    // ---- the split's partial: row n's max and sum (lane group 0) and its channels 16 nd + 4 g + i ----
    l_i = group_sum(l_i);
    if (!r_ok) return;
    float* slot = p.part + ((static_cast<int64_t>(prog) * p.splits + split) * 16 + n) * (DP + 2);
    if (g == 0) {
        slot[0] = m_i;
        slot[1] = l_i;
    }
#pragma unroll
    for (int nd = 0; nd < ND; ++nd)
#pragma unroll
        for (int i = 0; i < 4; ++i) slot[2 + 16 * nd + 4 * g + i] = acc[nd][i] * vs;
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

// One workgroup per (row, KV head, block of 16 query rows): per query row the largest split maximum M (and the sink
// logit), the sum sum_s l_s 2^(m_s - M), then every channel's sum_s acc_s 2^(m_s - M) over it (decode.py's merge,
// attention/_decode_kernels.py:183-226); zeros where nothing is visible.
template <int DP, int QF>
__global__ __launch_bounds__(256) void dense_merge_kernel(DenseParams p) {
    __shared__ float s_m[16], s_inv[16];
    const int prog = blockIdx.x;
    const int mt = prog % p.m_tiles;
    const int kvh = (prog / p.m_tiles) % p.kv_heads;
    const int b = prog / (p.m_tiles * p.kv_heads);
    const float* base = p.part + static_cast<int64_t>(prog) * p.splits * 16 * (DP + 2);
    const int t = static_cast<int>(threadIdx.x);
    if (t < 16) {
        const int r = mt * 16 + t;
        float big = -INFINITY;
        for (int s = 0; s < p.splits; ++s) big = fmaxf(big, base[(s * 16 + t) * (DP + 2)]);
        float sink = -INFINITY;
        if (p.sinks && r < p.rows) sink = p.sinks[kvh * p.groups + r / p.queries] * kLog2e;
        const float m = fmaxf(big, sink);
        float l = 0.0f;
        if (m != -INFINITY) {
            for (int s = 0; s < p.splits; ++s) {
                const float ms = base[(s * 16 + t) * (DP + 2)];
                if (ms != -INFINITY) l += base[(s * 16 + t) * (DP + 2) + 1] * __builtin_amdgcn_exp2f(ms - m);
            }
            if (sink != -INFINITY) l += __builtin_amdgcn_exp2f(sink - m);
        }
        s_m[t] = m;
        s_inv[t] = l > 0.0f ? 1.0f / l : 0.0f;
    }
    __syncthreads();
    for (int e = t; e < 16 * p.value_dim; e += blockDim.x) {
        const int rr = e / p.value_dim, d = e % p.value_dim;
        const int r = mt * 16 + rr;
        if (r >= p.rows) break;
        const float m = s_m[rr];
        float o = 0.0f;
        if (m != -INFINITY) {
            for (int s = 0; s < p.splits; ++s) {
                const float* slot = base + (s * 16 + rr) * (DP + 2);
                if (slot[0] != -INFINITY) o += slot[2 + d] * __builtin_amdgcn_exp2f(slot[0] - m);
            }
        }
        const int gq = r / p.queries, qi = r % p.queries;
        const int q_start = p.query_start_loc ? p.query_start_loc[b] : 0;
        if (p.query_start_loc && qi >= p.query_start_loc[b + 1] - q_start) continue;  // an inactive query row
        store_out<QF>(p, b * p.so_b + static_cast<int64_t>(q_start + qi) * p.so_q + (kvh * p.groups + gq) * p.so_h + d,
                      o * s_inv[rr]);
    }
}

template <int DP, int FMT, int QF>
int launch_dense(const DenseParams& p, hipStream_t stream) {
    const int programs = p.batch * p.kv_heads * p.m_tiles;
    hipLaunchKernelGGL((dense_split_kernel<DP, FMT, QF>), dim3(programs, p.splits), dim3(64), 0, stream, p);
    if (const int rc = check_launch("dense_split_kernel")) return rc;
    hipLaunchKernelGGL((dense_merge_kernel<DP, QF>), dim3(programs), dim3(256), 0, stream, p);
    return check_launch("dense_merge_kernel");
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
    return 0;
}

int dense_attention(const DenseParams& p, int padded_dim, hipStream_t stream) {
    switch (padded_dim) {
        case 64: return by_q_format<64>(p, stream);
        case 128: return by_q_format<128>(p, stream);
        case 256: return by_q_format<256>(p, stream);
        default: return fail("decode: head dims above 256 are not supported");
    }
}

}  // namespace eco
