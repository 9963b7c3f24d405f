// KIVI on vLLM's paged cell layout (the reference's backends/vllm/kivi/layout.py:1-21, 133-291 and kernels.py:58-78,
// 94-207): the cells of the tokens a request committed are quantized in place, bytewise as the reference's
// write_cells lays them out.
//
// quantize_committed: for every decoding request (not prefilling, a non-empty query, c = seq_len - query_len > 0
// tokens before the pass) and KV head, keys are quantized in whole groups of G tokens below (c / R) * R, newest first,
// until a group whose last cell is already quantized; values in tiles of 16 tokens below c - R, newest first, each
// token still full precision, until a tile held a quantized token. A quantized key group: per channel the fp32 min and
// max over its G tokens, scale = fp16r((max - min) / levels), zero = fp16r(min), codes round-half-even((x - zero) /
// safe) clamped (the quantize arithmetic of kivi_math.hpp, with IEEE divisions, the CPU definition the oracle pins);
// each dense entry becomes code * scale + zero (product, then sum) in the cache dtype, the codes are packed along the
// channels (8 / bits per byte, channel j pb + i at bit i bits), the 2D fp16 scales and zeros are spread over the
// group's cells (entry e in the cell of token s0 + e / ka, slot e % ka), and every cell's key flag becomes 1, or 2 when
// a scale or zero is beyond fp16. Values likewise per token over groups of vg channels, their nvg scales and zeros in
// the token's own cell. The walk's stopping points are found first over the flags as the pass finds them
// (kivi_cells_plan_kernel, one wave per (request, KV head)); the groups and tokens it covers are then quantized by
// many workgroups per row at once (a serial walk per row took 16.8 ms for 16 x 8192-token prompts).

#include <algorithm>

#include "common.hpp"
#include "kivi_cells.hpp"
#include "kivi_math.hpp"

namespace eco {

namespace {

constexpr int VT = 16;      // tokens per value tile
constexpr int MAX_D = 256;  // channels
constexpr int MAX_G = 128;  // tokens per key group

__device__ inline float load_value(const uint8_t* row, int d, int format) {
    if (format == BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(row)[d]);
    if (format == FP16) return static_cast<float>(reinterpret_cast<const _Float16*>(row)[d]);
    return reinterpret_cast<const float*>(row)[d];
}

__device__ inline void store_value(uint8_t* row, int d, int format, float x) {
    if (format == BF16)
        reinterpret_cast<uint16_t*>(row)[d] = f32_to_bf16(x);
    else if (format == FP16)
        reinterpret_cast<_Float16*>(row)[d] = static_cast<_Float16>(x);
    else
        reinterpret_cast<float*>(row)[d] = x;
}

__device__ inline void store_half(uint8_t* at, float x) { *reinterpret_cast<_Float16*>(at) = static_cast<_Float16>(x); }

// Byte offset of the cell of token t of request b at KV head kvh, or -1 when its page is not mapped.
__device__ inline int64_t cell_of(const CellsParams& p, int b, int kvh, int t) {
    const int lp = t / p.page_size;
    if (t < 0 || lp >= p.bt_cols) return -1;
    const int page = p.block_table[static_cast<int64_t>(b) * p.bt_stride + lp];
    if (page < 0 || page >= p.num_pages) return -1;
    return page * p.sb + kvh * p.sh + static_cast<int64_t>(t % p.page_size) * p.sn;
}

__device__ inline float dequantized(uint32_t code, const Quant& q) {
    return __fadd_rn(__fmul_rn(static_cast<float>(code), q.scale), q.low);
}

__device__ inline bool beyond_fp16(const Quant& q) { return fabsf(q.scale) > 65504.0f || fabsf(q.low) > 65504.0f; }

// The cells a request's pass quantizes, per (request, KV head), found before any cell changes (one wave): the walk
// of the reference goes newest first and stops at the first cell already quantized, which over the flags as they are
// when the pass starts is a search from the top. plan[4 (b Hkv + h) ..] = {k_lo, k_hi, v_lo, v_hi}: key groups
// [k_lo, k_hi) (groups of G tokens below (c / R) R, down to the group above the newest one whose last cell's key flag
// is set or is not mapped), value tokens [v_lo, v_hi) (tiles of VT tokens below c - R, newest first, down to and
// including the first tile that holds a token not to quantize: quantized, not mapped or before token 0; of these
// tokens, those whose value flag is clear).
__global__ __launch_bounds__(64) void kivi_cells_plan_kernel(CellsParams p, int32_t* plan) {
    const CellLayout& L = p.L;
    const int b = blockIdx.x, kvh = blockIdx.y, lane = threadIdx.x;
    const int G = L.group, R = p.residual;
    int32_t* out = plan + 4 * (static_cast<int64_t>(b) * p.kv_heads + kvh);
    const int qlen = p.query_start_loc[b + 1] - p.query_start_loc[b];
    const int c = p.seq_lens[b] - qlen;
    if (p.prefilling[b] != 0 || qlen <= 0 || c <= 0) {
        if (lane < 4) out[lane] = 0;
        return;
    }
    // keys: the newest group g below k_hi whose last cell is quantized or unmapped (g < 0: the walk's end)
    const int k_hi = (c / R) * R / G;
    int k_lo = 0;
    for (int top = k_hi - 1; top >= 0; top -= 64) {
        const int g = top - lane;
        bool stop = g < 0;
        if (!stop) {
            const int64_t last = cell_of(p, b, kvh, g * G + G - 1);
            stop = last < 0 || p.cache[last + L.off_flag] != 0;
        }
        const uint64_t hit = __ballot(stop);
        if (hit != 0) {
            k_lo = top - static_cast<int>(__builtin_ctzll(hit)) + 1;
            break;
        }
    }
    // values: tile i holds tokens top - VT (i + 1) .. top - VT i - 1 (top = c - R); the walk takes tiles while top -
    // VT i > 0 and stops after the first one holding a token not to quantize
    const int top = c - R;
    int v_lo = 0, v_hi = 0;
    if (top > 0) {
        v_hi = top;
        const int tiles = (top + VT - 1) / VT;
        int last = tiles - 1;  // the last tile the walk takes
        for (int i0 = 0; i0 < tiles; i0 += 64 / VT) {
            const int i = i0 + lane / VT;
            const int t = top - VT * (i + 1) + lane % VT;
            bool stop = false;
            if (i < tiles) {
                const int64_t cell = t >= 0 ? cell_of(p, b, kvh, t) : -1;
                stop = cell < 0 || p.cache[cell + L.off_flag + 1] != 0;
            }
            const uint64_t hit = __ballot(stop);
            if (hit != 0) {
                last = i0 + static_cast<int>(__builtin_ctzll(hit)) / VT;
                break;
            }
        }
        v_lo = max(top - VT * (last + 1), 0);
    }
    if (lane == 0) {
        out[0] = k_lo;
        out[1] = k_hi;
        out[2] = v_lo;
        out[3] = v_hi;
    }
}

// The pass's quantization after kivi_cells_plan_kernel (the next launch on the stream): workgroup (b, kvh, y) takes
// key groups k_lo + y, k_lo + y + Y, ... and value tiles of VT tokens v_lo + VT y, v_lo + VT (y + Y), ... (Y =
// gridDim.z); no two workgroups touch a cell, and the flags are written last for each group or token. A quantized key
// group: per channel the fp32 min and max over its G tokens, then codes, the dequantized dense entries, the 2D scales
// and zeros spread over the group's cells and every cell's key flag; a value token: per group of vg channels, in its
// own cell.
__global__ __launch_bounds__(256) void kivi_cells_quantize_kernel(CellsParams p, const int32_t* plan) {
    extern __shared__ uint8_t codes[];  // [max(G, VT)][D]
    __shared__ int s_over;
    __shared__ int s_todo[VT], s_tok_over[VT];
    __shared__ int64_t s_cell[VT];
    const CellLayout& L = p.L;
    const int b = blockIdx.x, kvh = blockIdx.y, y = blockIdx.z, Y = gridDim.z, tid = threadIdx.x;
    const int D = L.head_dim, G = L.group;
    const int levels = (1 << L.bits) - 1, pb = 8 / L.bits;
    const int32_t* range = plan + 4 * (static_cast<int64_t>(b) * p.kv_heads + kvh);
    const int k_lo = range[0], k_hi = range[1], v_lo = range[2], v_hi = range[3];

    // ---- keys ----
    for (int g = k_lo + y; g < k_hi; g += Y) {
        const int s0 = g * G;
        if (tid == 0) s_over = 0;
        __syncthreads();
        const int64_t base = cell_of(p, b, kvh, s0);  // a group lies in one page (pages hold whole groups)
        if (tid < D) {
            // the tokens' entries eight at a time, loaded together (the stores of a batch come after its loads)
            float lo = INFINITY, hi = -INFINITY;
            for (int t0 = 0; t0 < G; t0 += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    x[u] = t0 + u < G ? load_value(p.cache + base + (t0 + u) * p.sn, tid, p.format) : x[0];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    lo = __builtin_elementwise_minimum(lo, x[u]);  // NaN propagates, as torch's amin / amax
                    hi = __builtin_elementwise_maximum(hi, x[u]);
                }
            }
            const Quant q = make_quant(lo, hi, levels, nullptr);
            if (beyond_fp16(q)) atomicOr(&s_over, 1);
            for (int t0 = 0; t0 < G; t0 += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    x[u] = t0 + u < G ? load_value(p.cache + base + (t0 + u) * p.sn, tid, p.format) : 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (t0 + u >= G) break;
                    const uint32_t code = code_of(x[u], q, levels);
                    store_value(p.cache + base + (t0 + u) * p.sn, tid, p.format, dequantized(code, q));
                    codes[(t0 + u) * D + tid] = static_cast<uint8_t>(code);
                }
            }
            // aux entries tid (scale) and D + tid (zero point)
            store_half(p.cache + base + (tid / L.key_aux) * p.sn + L.off_ka + 2 * (tid % L.key_aux), q.scale);
            store_half(p.cache + base + ((D + tid) / L.key_aux) * p.sn + L.off_ka + 2 * ((D + tid) % L.key_aux),
                       q.low);
        }
        __syncthreads();
        const int bytes = D / pb;
        for (int j = tid; j < G * bytes; j += blockDim.x) {
            const int t = j / bytes, jj = j % bytes;
            uint32_t byte = 0;
            for (int i = 0; i < pb; ++i) byte |= static_cast<uint32_t>(codes[t * D + jj * pb + i]) << (i * L.bits);
            p.cache[base + t * p.sn + L.off_kc + jj] = static_cast<uint8_t>(byte);
        }
        if (tid < G) p.cache[base + tid * p.sn + L.off_flag] = static_cast<uint8_t>(1 + s_over);
        __syncthreads();
    }

    // ---- values ----
    const int vg = L.value_group, nvg = D / vg;
    for (int t0 = v_lo + VT * y; t0 < v_hi; t0 += VT * Y) {
        if (tid < VT) {
            const int t = t0 + tid;
            const int64_t cell = t < v_hi ? cell_of(p, b, kvh, t) : -1;
            s_cell[tid] = cell;
            s_todo[tid] = cell >= 0 && p.cache[cell + L.off_flag + 1] == 0;
            s_tok_over[tid] = 0;
        }
        __syncthreads();
        for (int item = tid; item < VT * nvg; item += blockDim.x) {
            const int tt = item / nvg, j = item % nvg;
            if (!s_todo[tt]) continue;
            uint8_t* row = p.cache + s_cell[tt] + L.off_v;
            float lo = INFINITY, hi = -INFINITY;
            for (int e0 = 0; e0 < vg; e0 += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) x[u] = e0 + u < vg ? load_value(row, j * vg + e0 + u, p.format) : x[0];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    lo = __builtin_elementwise_minimum(lo, x[u]);
                    hi = __builtin_elementwise_maximum(hi, x[u]);
                }
            }
            const Quant q = make_quant(lo, hi, levels, nullptr);
            if (beyond_fp16(q)) atomicOr(&s_tok_over[tt], 1);
            for (int e0 = 0; e0 < vg; e0 += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) x[u] = e0 + u < vg ? load_value(row, j * vg + e0 + u, p.format) : 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (e0 + u >= vg) break;
                    const uint32_t code = code_of(x[u], q, levels);
                    store_value(row, j * vg + e0 + u, p.format, dequantized(code, q));
                    codes[tt * D + j * vg + e0 + u] = static_cast<uint8_t>(code);
                }
            }
            store_half(p.cache + s_cell[tt] + L.off_vs + 2 * j, q.scale);
            store_half(p.cache + s_cell[tt] + L.off_vz + 2 * j, q.low);
        }
        __syncthreads();
        const int bytes = D / pb;
        for (int j = tid; j < VT * bytes; j += blockDim.x) {
            const int tt = j / bytes, jj = j % bytes;
            if (!s_todo[tt]) continue;
            uint32_t byte = 0;
            for (int i = 0; i < pb; ++i) byte |= static_cast<uint32_t>(codes[tt * D + jj * pb + i]) << (i * L.bits);
            p.cache[s_cell[tt] + L.off_vc + jj] = static_cast<uint8_t>(byte);
        }
        if (tid < VT && s_todo[tid]) p.cache[s_cell[tid] + L.off_flag + 1] = static_cast<uint8_t>(1 + s_tok_over[tid]);
        __syncthreads();
    }
}

// The cells vLLM's cache write just filled are full precision: both flags of every head cleared.
__global__ void kivi_cells_clear_kernel(CellsParams p, const int32_t* slots) {
    const int slot = slots[blockIdx.x];
    if (slot < 0 || slot / p.page_size >= p.num_pages) return;
    for (int h = threadIdx.x; h < p.kv_heads; h += blockDim.x) {
        uint8_t* cell = p.cache + (slot / p.page_size) * p.sb + h * p.sh + static_cast<int64_t>(slot % p.page_size) * p.sn;
        cell[p.L.off_flag] = 0;
        cell[p.L.off_flag + 1] = 0;
    }
}

}  // namespace

int kivi_cells_quantize(const CellsParams& p, int32_t* plan, hipStream_t stream) {
    if (p.requests == 0 || p.kv_heads == 0) return 0;
    if (p.L.head_dim > MAX_D || p.L.group > MAX_G)
        return fail("kivi cells: head dims up to 256 and groups up to 128 tokens");
    hipLaunchKernelGGL(kivi_cells_plan_kernel, dim3(p.requests, p.kv_heads), dim3(64), 0, stream, p, plan);
    if (int rc = check_launch("kivi_cells_plan_kernel")) return rc;
    // about 4096 workgroups over the (request, KV head) rows, at most 64 per row
    const int rows = p.requests * p.kv_heads;
    const int per_row = std::max(1, std::min(64, 4096 / std::max(rows, 1)));
    const size_t lds = static_cast<size_t>(std::max(p.L.group, VT)) * p.L.head_dim;  // the codes of a group or tile
    hipLaunchKernelGGL(kivi_cells_quantize_kernel, dim3(p.requests, p.kv_heads, per_row), dim3(256), lds, stream, p,
                       plan);
    return check_launch("kivi_cells_quantize_kernel");
}

int kivi_cells_clear_flags(const CellsParams& p, const int32_t* slots, int tokens, hipStream_t stream) {
    if (tokens == 0) return 0;
    hipLaunchKernelGGL(kivi_cells_clear_kernel, dim3(tokens), dim3(64), 0, stream, p, slots);
    return check_launch("kivi_cells_clear_kernel");
}

}  // namespace eco
