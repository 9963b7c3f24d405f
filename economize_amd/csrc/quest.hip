// Quest page bounds and query-aware page selection (gfx950).
//
// Page bounds follow page_bounds (attention/quest.py:54-65): the channel-wise smallest and largest key of every page,
// fp8 keys decoded exactly (bf16 holds every fp8 value), written as bf16 (fp16 and fp32 keys of a dense buffer: in
// their own format, as bounds_dtype, attention/quest.py:68-70). They are computed from the stored cache
// elements; a per-head fp8 scale is positive and multiplies every score of a (row, KV head) alike, so it does not
// change which pages are selected and is not applied.
//
// Selection follows select_pages (attention/quest.py:73-108):
//   score[b, h, p] = sum_d qsum_d (lo_pd + hi_pd) / 2 + sum_d qabs_d (hi_pd - lo_pd) / 2
// with qsum / qabs the fp32 sums of q / |q| over the KV head's query rows (rows r = g * Q + qi added in order),
// pages at or past done[b] excluded, the top min(pages, max_done) pages, increasing, then -1. The reference leaves
// two things open that are fixed here (and in the oracle): the fp32 order of the two dot products (products rounded
// to fp32, sequential sums over runs of 8 channels, then a halving tree over the runs, run j plus run j + n / 2, n
// the run count padded to a power of two) and ties (equal scores are taken lowest page first).
//
// Kernels: quest_bounds_kernel (one wave per row, Quest page and KV head, over the paged cache),
// quest_dense_bounds_kernel (the same over a dense key buffer of any format), quest_score_kernel (a chunk of pages of
// one (row, KV head) per workgroup: the bounds are the bytes a selection reads, so the scoring is spread over the
// whole chip), quest_topk_kernel (one workgroup per (row, KV head): a radix select over order-preserving integer keys
// of the scores, ties to the lower index, then a compaction in page order).

#include <type_traits>

#include "common.hpp"
#include "quest.hpp"
#include "quest_page.hpp"

namespace eco {

namespace {

constexpr int SCORE_PASSES = 4;  // pages per scoring thread

// Scores of a (row, KV head) in the workspace: max_done floats, rows 16-byte aligned.
__host__ __device__ inline int64_t score_stride(int max_done) { return (max_done + 3) & ~3; }
constexpr int TOPK_LDS_KEYS = 15360;  // rows of at most this many committed pages select from keys held in LDS (60 KiB)

// One wave per (row b, Quest page first + i, KV head).
template <int FMT>
__global__ __launch_bounds__(64) void quest_bounds_kernel(BoundsParams p) {
    const int pages = p.last - p.first;
    quest_bounds_of_page<FMT>(p, blockIdx.x / pages, p.first + blockIdx.x % pages, blockIdx.y, threadIdx.x);
}

// The bounds of the pages each (row, KV head) committed since its last refresh, with every range on the device (a
// launch of fixed shape, so a decode step that keeps its Quest metadata can be captured in a graph): workgroup
// (b * Hkv + h, y) takes pages valid + y, valid + y + Y, ... below the row's committed pages.
template <int FMT>
__global__ __launch_bounds__(64) void quest_refresh_kernel(BoundsParams p) {
    const int row = blockIdx.x;
    const int b = row / p.kv_heads, kvh = row % p.kv_heads;
    const int last = min(max(p.committed[b], 0) / (16 * p.span), p.page_cap);
    for (int qp = p.valid[row] + static_cast<int>(blockIdx.y); qp < last; qp += gridDim.y)
        quest_bounds_of_page<FMT>(p, b, qp, kvh, threadIdx.x);
}

// After quest_refresh_kernel (the next launch on the stream): the refreshed pages are final, and done[b] is the
// row's committed Quest pages.
__global__ void quest_mark_kernel(BoundsParams p) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= p.batch * p.kv_heads) return;
    const int b = row / p.kv_heads;
    const int last = min(max(p.committed[b], 0) / (16 * p.span), p.page_cap);
    p.valid[row] = max(p.valid[row], last);
    if (p.done && row % p.kv_heads == 0) p.done[b] = last;
}

// One key element of format KF as fp32 (exact; fp8 decoded by the hardware converter at scale 1).
template <int KF>
__device__ inline float key_f32(const uint8_t* base, int64_t i) {
    if constexpr (KF == BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
    if constexpr (KF == FP16) return static_cast<float>(reinterpret_cast<const _Float16*>(base)[i]);
    if constexpr (KF == FP32) return reinterpret_cast<const float*>(base)[i];
    if constexpr (KF == FP8_E4M3) return __builtin_amdgcn_cvt_scalef32_f32_fp8(base[i], 1.0f, 0);
    return __builtin_amdgcn_cvt_scalef32_f32_bf8(base[i], 1.0f, 0);
}

// The bounds of pages [first, last) of a dense key buffer, one wave per (row, page, KV head): lane l takes channels
// l, l + 64, ... and walks the page's slots (adjacent lanes read adjacent channels of one slot). Minimum and maximum
// propagate NaN, as torch's amin / amax do; the results are exact in the bounds' format (bf16 holds every bf16 and
// fp8 value, fp16 and fp32 keys keep their own format).
template <int KF, int BF>
__global__ __launch_bounds__(64) void quest_dense_bounds_kernel(DenseBoundsParams p) {
    const int pages = p.last - p.first;
    const int b = blockIdx.x / pages;
    const int pg = p.first + blockIdx.x % pages;
    const int kvh = blockIdx.y;
    const uint8_t* keys = static_cast<const uint8_t*>(p.keys);
    const int64_t base = b * p.sk_b + kvh * p.sk_h + static_cast<int64_t>(pg) * p.page * p.sk_s;
    for (int c = threadIdx.x; c < p.head_dim; c += 64) {
        float lo = INFINITY, hi = -INFINITY;
        for (int t = 0; t < p.page; ++t) {
            const float x = key_f32<KF>(keys, base + static_cast<int64_t>(t) * p.sk_s + c);
            lo = __builtin_elementwise_minimum(lo, x);
            hi = __builtin_elementwise_maximum(hi, x);
        }
        const int64_t at = b * p.sb_b + kvh * p.sb_h + static_cast<int64_t>(pg) * p.sb_p + c;
        if constexpr (BF == BF16) {
            static_cast<uint16_t*>(p.kmin)[at] = f32_to_bf16(lo);
            static_cast<uint16_t*>(p.kmax)[at] = f32_to_bf16(hi);
        } else if constexpr (BF == FP16) {
            static_cast<_Float16*>(p.kmin)[at] = static_cast<_Float16>(lo);
            static_cast<_Float16*>(p.kmax)[at] = static_cast<_Float16>(hi);
        } else {
            static_cast<float*>(p.kmin)[at] = lo;
            static_cast<float*>(p.kmax)[at] = hi;
        }
    }
}

// One element of a query or of page bounds as fp32 (exact): bf16, fp16 or fp32.
template <int F>
__device__ inline float elem_f32(const void* base, int64_t i) {
    if constexpr (F == BF16) return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
    if constexpr (F == FP16) return static_cast<float>(static_cast<const _Float16*>(base)[i]);
    return static_cast<const float*>(base)[i];
}

// Eight consecutive bounds (16-byte words: one for bf16 / fp16, two for fp32) as fp32.
template <int BF>
__device__ inline float bound_of(const uint4 (&w)[BF == FP32 ? 2 : 1], int i) {
    if constexpr (BF == FP32) {
        const uint4 x = w[i >> 2];
        const uint32_t u = (i & 3) == 0 ? x.x : ((i & 3) == 1 ? x.y : ((i & 3) == 2 ? x.z : x.w));
        return bits_f32(u);
    } else {
        const uint32_t words[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
        const uint16_t h = static_cast<uint16_t>(words[i >> 1] >> (16 * (i & 1)));
        if constexpr (BF == BF16) return bf16_to_f32(h);
        return static_cast<float>(__builtin_bit_cast(_Float16, h));
    }
}

// Scores of pages [chunk * blockIdx.x, +chunk) of row (b, kvh) = blockIdx.y: L lanes per page (L = the run count
// padded to a power of two), lane j holding channels 8 j .. 8 j + 7; a workgroup covers SCORE_PASSES * 256 / L
// pages, and every thread issues the bound loads of all its pages before it sums the query rows. QF / BF: the
// formats of the query and of the bounds (bf16, fp16, fp32), both widened exactly to fp32.
template <int QF, int BF>
__global__ __launch_bounds__(256) void quest_score_kernel(SelectParams p) {
    constexpr int BW = BF == FP32 ? 2 : 1;  // 16-byte words per 8 bounds
    constexpr int BES = BF == FP32 ? 4 : 2;
    __shared__ float qsum[512], qabs[512];
    const int row = blockIdx.y;
    const int b = row / p.kv_heads;
    const int kvh = row % p.kv_heads;
    const int rows = p.groups * p.queries;
    const int runs = p.head_dim / 8;
    int L = 1;
    while (L < runs) L <<= 1;
    const int per_pass = blockDim.x / L;
    const int j = threadIdx.x % L;
    const int done = min(max(p.done[b], 0), p.max_done);
    const int p0 = blockIdx.x * p.chunk;
    const int p1 = min(p0 + p.chunk, p.max_done);
    uint4 lw[SCORE_PASSES][BW], hw[SCORE_PASSES][BW];
#pragma unroll
    for (int k = 0; k < SCORE_PASSES; ++k) {
        const int page = p0 + k * per_pass + static_cast<int>(threadIdx.x) / L;
#pragma unroll
        for (int w = 0; w < BW; ++w) lw[k][w] = hw[k][w] = make_uint4(0, 0, 0, 0);
        if (page < p1 && j < runs) {
            const int64_t at = b * p.sb_b + kvh * p.sb_h + static_cast<int64_t>(page) * p.sb_p + 8 * j;
            // the bounds are read once per selection: streamed loads
#pragma unroll
            for (int w = 0; w < BW; ++w) {
                lw[k][w] = stream_load16(static_cast<const uint8_t*>(p.kmin) + at * BES + 16 * w);
                hw[k][w] = stream_load16(static_cast<const uint8_t*>(p.kmax) + at * BES + 16 * w);
            }
        }
    }
    for (int d = threadIdx.x; d < p.head_dim; d += blockDim.x) {
        float s = 0.0f, a = 0.0f;
        // rows added in order; the loads of 8 rows are in flight together
        for (int r0 = 0; r0 < rows; r0 += 8) {
            float x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int r = r0 + u < rows ? r0 + u : r0;
                const int g = r / p.queries, qi = r % p.queries;
                x[u] = elem_f32<QF>(p.q, b * p.sq_b + qi * p.sq_q + (kvh * p.groups + g) * p.sq_h + d);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (r0 + u >= rows) break;
                s = r0 + u == 0 ? x[u] : s + x[u];
                a = r0 + u == 0 ? fabsf(x[u]) : a + fabsf(x[u]);
            }
        }
        qsum[d] = s;
        qabs[d] = a;
    }
    __syncthreads();
    float* out = p.scores + static_cast<int64_t>(row) * score_stride(p.max_done);
#pragma unroll
    for (int k = 0; k < SCORE_PASSES; ++k) {
        const int page = p0 + k * per_pass + static_cast<int>(threadIdx.x) / L;
        float s1 = 0.0f, s2 = 0.0f;
        if (j < runs) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float lo = bound_of<BF>(lw[k], i);
                const float hi = bound_of<BF>(hw[k], i);
                const float mid = (lo + hi) * 0.5f;
                const float half = (hi - lo) * 0.5f;
                const float t1 = qsum[8 * j + i] * mid;
                const float t2 = qabs[8 * j + i] * half;
                s1 = i == 0 ? t1 : s1 + t1;
                s2 = i == 0 ? t2 : s2 + t2;
            }
        }
        if (L == 16) {
            // the halving tree over a DPP row: lane j < off adds lane j + off (row_shl), which for lane 0 is the
            // xor tree below, term for term
            auto fold = [&](float& x, auto ctrl) __attribute__((always_inline)) {
                x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                           decltype(ctrl)::value, 0xF, 0xF, false));
            };
            using std::integral_constant;
            fold(s1, integral_constant<int, 0x108>{});  // row_shl:8
            fold(s2, integral_constant<int, 0x108>{});
            fold(s1, integral_constant<int, 0x104>{});  // row_shl:4
            fold(s2, integral_constant<int, 0x104>{});
            fold(s1, integral_constant<int, 0x102>{});  // row_shl:2
            fold(s2, integral_constant<int, 0x102>{});
            fold(s1, integral_constant<int, 0x101>{});  // row_shl:1
            fold(s2, integral_constant<int, 0x101>{});
        } else {
            for (int off = L / 2; off > 0; off >>= 1) {
                s1 += __shfl_xor(s1, off);
                s2 += __shfl_xor(s2, off);
            }
        }
        if (page < p1 && j == 0)
            out[page] = page < done ? (page == 0 && p.first_page ? INFINITY : s1 + s2) : -INFINITY;
    }
}

// Order-preserving integer key of a score (a larger score has a larger key; -0 counts as +0).
__device__ inline uint32_t score_key(float x) {
    const uint32_t u = f32_bits(x == 0.0f ? 0.0f : x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive scan over a wave by DPP: within rows of 16 lanes by row shifts of 1, 2, 4 and 8 (a lane shifted in from
// outside the row adds the 0 of the old operand), then across rows: row_bcast:15 adds lane 15 of rows 0 and 2 to rows
// 1 and 3, row_bcast:31 adds lane 31 (the total of rows 0 and 1) to rows 2 and 3.
__device__ inline int wave_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return x;
}

// The largest and smallest value over a wave (by the same DPP pattern as wave_scan; lane 63 ends with the result).
__device__ inline uint32_t wave_max_u32(uint32_t x) {
    auto step = [&](auto ctrl, auto rows) __attribute__((always_inline)) {
        const uint32_t y = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            0, static_cast<int>(x), decltype(ctrl)::value, decltype(rows)::value, 0xF, false));
        x = x > y ? x : y;
    };
    using std::integral_constant;
    step(integral_constant<int, 0x111>{}, integral_constant<int, 0xF>{});  // row_shr:1
    step(integral_constant<int, 0x112>{}, integral_constant<int, 0xF>{});  // row_shr:2
    step(integral_constant<int, 0x114>{}, integral_constant<int, 0xF>{});  // row_shr:4
    step(integral_constant<int, 0x118>{}, integral_constant<int, 0xF>{});  // row_shr:8
    step(integral_constant<int, 0x142>{}, integral_constant<int, 0xA>{});  // row_bcast:15
    step(integral_constant<int, 0x143>{}, integral_constant<int, 0xC>{});  // row_bcast:31
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 63));
}

__device__ inline uint32_t wave_min_u32(uint32_t x) {
    auto step = [&](auto ctrl, auto rows) __attribute__((always_inline)) {
        const uint32_t y = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            -1, static_cast<int>(x), decltype(ctrl)::value, decltype(rows)::value, 0xF, false));
        x = x < y ? x : y;
    };
    using std::integral_constant;
    step(integral_constant<int, 0x111>{}, integral_constant<int, 0xF>{});  // row_shr:1
    step(integral_constant<int, 0x112>{}, integral_constant<int, 0xF>{});  // row_shr:2
    step(integral_constant<int, 0x114>{}, integral_constant<int, 0xF>{});  // row_shr:4
    step(integral_constant<int, 0x118>{}, integral_constant<int, 0xF>{});  // row_shr:8
    step(integral_constant<int, 0x142>{}, integral_constant<int, 0xA>{});  // row_bcast:15
    step(integral_constant<int, 0x143>{}, integral_constant<int, 0xC>{});  // row_bcast:31
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 63));
}

// Inclusive scan of one value per thread over a 256-thread workgroup; *total receives the sum.
__device__ inline int block_scan(int x, int* lds4, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    x = wave_scan(x);
    if (lane == 63) lds4[wave] = x;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += lds4[w];
    *total = lds4[0] + lds4[1] + lds4[2] + lds4[3];
    __syncthreads();
    return x + before;
}

// Inclusive scans of two values per thread over a 256-thread workgroup, through one exchange (lds8: 8 ints).
__device__ inline int2 block_scan2(int x, int y, int* lds8) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    x = wave_scan(x);
    y = wave_scan(y);
    if (lane == 63) {
        lds8[wave] = x;
        lds8[4 + wave] = y;
    }
    __syncthreads();
    int bx = 0, by = 0;
    for (int w = 0; w < wave; ++w) {
        bx += lds8[w];
        by += lds8[4 + w];
    }
    __syncthreads();
    return make_int2(x + bx, y + by);
}

// One workgroup of 256 threads per (row, KV head): the top `count` of the row's committed pages by score, written in
// increasing page order, then -1. With IN_LDS the row's keys are read from global memory once, into LDS; otherwise
// (rows of more than TOPK_LDS_KEYS pages) every pass reads them from global memory again.
template <bool IN_LDS>
__global__ __launch_bounds__(256) void quest_topk_kernel(SelectParams p) {
    extern __shared__ uint32_t lds_keys[];
    __shared__ int hist[2048];
    __shared__ __align__(16) uint32_t cand[256];
    __shared__ int lds4[4], lds8[8];
    __shared__ uint32_t shared_prefix, red[8];
    __shared__ int shared_rem, shared_m, shared_d, cand_count;
    const int row = blockIdx.x;
    const int b = row / p.kv_heads;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const float* scores = p.scores + static_cast<int64_t>(row) * score_stride(p.max_done);
    if constexpr (IN_LDS) {
        // every page below max_done has a score (-inf from done on): the loads go out with the read of done[b]
#pragma unroll 8
        for (int i = t; i < p.max_done; i += 256) lds_keys[i] = score_key(scores[i]);
    }
    const int n = min(max(p.done[b], 0), p.max_done);
    const int count = min(p.pages, p.max_done);
    int32_t* out = p.out + static_cast<int64_t>(row) * p.pages;
    int total = 0;
    if (n <= count || count <= 0) {  // every committed page (or none to select)
        for (int i = t; i < p.pages; i += 256) out[i] = i < n ? i : -1;
        return;
    }
    if constexpr (IN_LDS) __syncthreads();
    auto key_at = [&](int i) __attribute__((always_inline)) -> uint32_t {
        if constexpr (IN_LDS)
            return lds_keys[i];
        else
            return score_key(scores[i]);
    };
    // Selection of the count-th largest key (the threshold) and of how many keys equal to it are taken (rem). The
    // keys at issue lie in [lo_k, hi_k], at first every key. A pass counts them into 2048 buckets by a monotone map
    // of the key over the interval and finds the bucket holding the rem-th largest; when it has at most 256 keys,
    // they are gathered and ranked against each other, which fixes the threshold; otherwise the interval shrinks to
    // that bucket's smallest and largest key (the interval's own smallest or largest key always falls outside it)
    // until it holds one key value. Histograms visit keys in any order; ties are settled by the compaction below.
    auto block_min_max = [&](uint32_t mn, uint32_t mx, uint32_t& lo_out, uint32_t& hi_out) __attribute__((always_inline)) {
        mn = wave_min_u32(mn);
        mx = wave_max_u32(mx);
        const int wave = t >> 6;
        if (lane == 0) {
            red[wave] = mn;
            red[4 + wave] = mx;
        }
        __syncthreads();
        lo_out = min(min(red[0], red[1]), min(red[2], red[3]));
        hi_out = max(max(red[4], red[5]), max(red[6], red[7]));
        __syncthreads();
    };
    uint32_t lo_k, hi_k;
    {
        uint32_t mn = 0xFFFFFFFFu, mx = 0u;
        for (int i = t; i < n; i += 256) {
            const uint32_t key = key_at(i);
            mn = min(mn, key);
            mx = max(mx, key);
        }
        if (t == 0) cand_count = 0;
        block_min_max(mn, mx, lo_k, hi_k);
    }
    int rem = count;
    uint32_t prefix = lo_k;  // the threshold
    while (lo_k != hi_k) {
        const float scale = 2048.0f / (static_cast<float>(hi_k - lo_k) + 1.0f);
        const uint32_t lo = lo_k, hi = hi_k;
        auto bucket = [&](uint32_t key) __attribute__((always_inline)) {
            return min(2047, static_cast<int>(static_cast<float>(key - lo) * scale));
        };
        for (int d = t; d < 2048; d += 256) hist[d] = 0;
        __syncthreads();
        for (int i0 = t - lane; i0 < n; i0 += 256) {
            // the wave's keys of this round: lanes whose bucket equals the first matching lane's add as one
            const int i = i0 + lane;
            const uint32_t key = i < n ? key_at(i) : 0u;
            const bool match = i < n && key >= lo && key <= hi;
            const int digit = match ? bucket(key) : 0;
            const uint64_t matching = __ballot(match);
            if (matching == 0) continue;
            const int leader = __builtin_ctzll(matching);
            const int lead_digit = __builtin_amdgcn_readlane(digit, leader);
            const uint64_t same = __ballot(match && digit == lead_digit);
            if (lane == leader) atomicAdd(&hist[lead_digit], static_cast<int>(__popcll(same)));
            if (match && digit != lead_digit) atomicAdd(&hist[digit], 1);
        }
        __syncthreads();
        int c = 0;  // thread t holds the buckets 2047 - 8 t down to 2040 - 8 t
#pragma unroll
        for (int k = 0; k < 8; ++k) c += hist[2047 - 8 * t - k];
        const int incl = block_scan(c, lds4, &total);
        if (incl >= rem && incl - c < rem) {
            int cum = incl - c;
            for (int k = 0; k < 8; ++k) {
                const int d = 2047 - 8 * t - k;
                if (cum + hist[d] >= rem) {
                    shared_d = d;
                    shared_rem = rem - cum;
                    shared_m = hist[d];
                    break;
                }
                cum += hist[d];
            }
        }
        __syncthreads();
        const int d = shared_d, m = shared_m;
        rem = shared_rem;
        if (m <= 256) {
            for (int i = t; i < n; i += 256) {
                const uint32_t key = key_at(i);
                if (key >= lo && key <= hi && bucket(key) == d) cand[atomicAdd(&cand_count, 1)] = key;  // m slots
            }
            __syncthreads();
            if (t < m) {  // the candidate whose rank range holds rem is the threshold
                const uint32_t mine = cand[t];
                int gt = 0, ge = 0;
#pragma unroll 4
                for (int j = 0; j < m; j += 4) {  // four candidates per LDS read (slots from m on are not counted)
                    const uint4 o = reinterpret_cast<const uint4*>(cand)[j / 4];
                    const uint32_t others[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const bool in = j + e < m;
                        gt += in && others[e] > mine ? 1 : 0;
                        ge += in && others[e] >= mine ? 1 : 0;
                    }
                }
                if (gt < rem && rem <= ge) {
                    shared_prefix = mine;
                    shared_rem = rem - gt;
                }
            }
            __syncthreads();
            prefix = shared_prefix;
            rem = shared_rem;
            break;
        }
        uint32_t mn = 0xFFFFFFFFu, mx = 0u;
        for (int i = t; i < n; i += 256) {
            const uint32_t key = key_at(i);
            if (key >= lo && key <= hi && bucket(key) == d) {
                mn = min(mn, key);
                mx = max(mx, key);
            }
        }
        block_min_max(mn, mx, lo_k, hi_k);
        prefix = lo_k;
    }
    // keys above the threshold, and the first `rem` keys equal to it in page order: thread t takes a contiguous range
    // of `per` keys, held in registers when there are at most 8
    const int per = (n + 255) / 256;
    const int i0 = min(t * per, n), i1 = min(i0 + per, n);
    auto compact = [&](auto cache_tag) __attribute__((always_inline)) {
        constexpr int C = decltype(cache_tag)::value;  // keys held in registers (0: read at every use)
        uint32_t held[C > 0 ? C : 1];
        if constexpr (C > 0) {
#pragma unroll
            for (int k = 0; k < C; ++k) held[k] = i0 + k < i1 ? key_at(i0 + k) : 0u;
        }
        const int span = C > 0 ? C : i1 - i0;
        auto key_of = [&](int k) __attribute__((always_inline)) { return C > 0 ? held[k] : key_at(i0 + k); };
        // one scan of the thread's keys above the threshold and of those equal to it: the threads before t hold
        // keys above it, all taken, and eq_before equal ones, of which the first rem are taken
        int eq = 0, above = 0;
#pragma unroll
        for (int k = 0; k < span; ++k) {
            if (i0 + k >= i1) continue;
            const uint32_t key = key_of(k);
            eq += key == prefix ? 1 : 0;
            above += key > prefix ? 1 : 0;
        }
        const int2 incl = block_scan2(above, eq, lds8);
        const int eq_before = incl.y - eq;
        const int eq_taken = min(max(rem - eq_before, 0), eq);  // this thread's first eq_taken equal keys
        int pos = incl.x - above + min(eq_before, rem);
        int e = 0;
#pragma unroll
        for (int k = 0; k < span; ++k) {
            if (i0 + k >= i1) continue;
            const uint32_t key = key_of(k);
            bool take = key > prefix;
            if (key == prefix) take = e++ < eq_taken;
            if (take) out[pos++] = i0 + k;
        }
    };
    if (per <= 8)
        compact(std::integral_constant<int, 8>{});
    else
        compact(std::integral_constant<int, 0>{});
    for (int i = count + t; i < p.pages; i += 256) out[i] = -1;
}

}  // namespace

int quest_score_chunk(int head_dim) {
    int L = 1;
    while (L < head_dim / 8) L <<= 1;
    return SCORE_PASSES * 256 / L;
}

int quest_bounds(const BoundsParams& p, hipStream_t stream) {
    if (p.last <= p.first) return 0;
    dim3 grid(static_cast<unsigned>(p.batch) * (p.last - p.first), p.kv_heads);
    switch (p.kv_format) {
        case BF16: hipLaunchKernelGGL(quest_bounds_kernel<BF16>, grid, dim3(64), 0, stream, p); break;
        case FP8_E4M3: hipLaunchKernelGGL(quest_bounds_kernel<FP8_E4M3>, grid, dim3(64), 0, stream, p); break;
        case FP8_E5M2: hipLaunchKernelGGL(quest_bounds_kernel<FP8_E5M2>, grid, dim3(64), 0, stream, p); break;
        default: return fail("quest page bounds: KV format must be bf16, fp8 e4m3 or fp8 e5m2");
    }
    return check_launch("quest_bounds_kernel");
}

int quest_dense_bounds(const DenseBoundsParams& p, hipStream_t stream) {
    if (p.last <= p.first) return 0;
    dim3 grid(static_cast<unsigned>(p.batch) * (p.last - p.first), p.kv_heads);
    switch (p.kv_format) {
        case BF16: hipLaunchKernelGGL((quest_dense_bounds_kernel<BF16, BF16>), grid, dim3(64), 0, stream, p); break;
        case FP16: hipLaunchKernelGGL((quest_dense_bounds_kernel<FP16, FP16>), grid, dim3(64), 0, stream, p); break;
        case FP32: hipLaunchKernelGGL((quest_dense_bounds_kernel<FP32, FP32>), grid, dim3(64), 0, stream, p); break;
        case FP8_E4M3:
            hipLaunchKernelGGL((quest_dense_bounds_kernel<FP8_E4M3, BF16>), grid, dim3(64), 0, stream, p);
            break;
        case FP8_E5M2:
            hipLaunchKernelGGL((quest_dense_bounds_kernel<FP8_E5M2, BF16>), grid, dim3(64), 0, stream, p);
            break;
        default: return fail("quest page bounds: keys must be bf16, fp16, fp32, fp8 e4m3 or fp8 e5m2");
    }
    return check_launch("quest_dense_bounds_kernel");
}

int quest_refresh(const BoundsParams& p, hipStream_t stream) {
    const int rows = p.batch * p.kv_heads;
    if (rows == 0) return 0;
    constexpr int CHUNKS = 8;  // waves per (row, KV head): a decode step completes at most one page per row
    dim3 grid(rows, CHUNKS);
    switch (p.kv_format) {
        case BF16: hipLaunchKernelGGL(quest_refresh_kernel<BF16>, grid, dim3(64), 0, stream, p); break;
        case FP8_E4M3: hipLaunchKernelGGL(quest_refresh_kernel<FP8_E4M3>, grid, dim3(64), 0, stream, p); break;
        case FP8_E5M2: hipLaunchKernelGGL(quest_refresh_kernel<FP8_E5M2>, grid, dim3(64), 0, stream, p); break;
        default: return fail("quest refresh: KV format must be bf16, fp8 e4m3 or fp8 e5m2");
    }
    if (int rc = check_launch("quest_refresh_kernel")) return rc;
    hipLaunchKernelGGL(quest_mark_kernel, dim3((rows + 255) / 256), dim3(256), 0, stream, p);
    return check_launch("quest_mark_kernel");
}

int quest_select(const SelectParams& p, hipStream_t stream) {
    const int rows = p.batch * p.kv_heads;
    if (p.max_done > 0) {
        if (p.chunk != quest_score_chunk(p.head_dim)) return fail("quest select: score chunk does not match the head dim");
        dim3 grid((p.max_done + p.chunk - 1) / p.chunk, rows);
        auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, p); };
        const int formats = p.q_format * 8 + p.bounds_format;
        switch (formats) {
            case BF16 * 8 + BF16: launch(quest_score_kernel<BF16, BF16>); break;
            case BF16 * 8 + FP16: launch(quest_score_kernel<BF16, FP16>); break;
            case BF16 * 8 + FP32: launch(quest_score_kernel<BF16, FP32>); break;
            case FP16 * 8 + BF16: launch(quest_score_kernel<FP16, BF16>); break;
            case FP16 * 8 + FP16: launch(quest_score_kernel<FP16, FP16>); break;
            case FP16 * 8 + FP32: launch(quest_score_kernel<FP16, FP32>); break;
            case FP32 * 8 + BF16: launch(quest_score_kernel<FP32, BF16>); break;
            case FP32 * 8 + FP16: launch(quest_score_kernel<FP32, FP16>); break;
            case FP32 * 8 + FP32: launch(quest_score_kernel<FP32, FP32>); break;
            default: return fail("quest select: queries and bounds must be bf16, fp16 or fp32");
        }
        if (int rc = check_launch("quest_score_kernel")) return rc;
    }
    if (p.max_done <= TOPK_LDS_KEYS) {
        const size_t lds = static_cast<size_t>(p.max_done > 0 ? p.max_done : 1) * sizeof(uint32_t);
        hipLaunchKernelGGL(quest_topk_kernel<true>, dim3(rows), dim3(256), lds, stream, p);
    } else {
        hipLaunchKernelGGL(quest_topk_kernel<false>, dim3(rows), dim3(256), 0, stream, p);
    }
    return check_launch("quest_topk_kernel");
}

}  // namespace eco
