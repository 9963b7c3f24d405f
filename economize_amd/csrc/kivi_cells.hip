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
// the token's own cell. One workgroup per (request, KV head); O(quantized tokens) bytes, off the decode path.

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

__global__ __launch_bounds__(256) void kivi_cells_quantize_kernel(CellsParams p) {
    __shared__ uint8_t codes[MAX_G * MAX_D];
    __shared__ int s_flag, s_over;
    __shared__ int s_todo[VT], s_tok_over[VT];
    __shared__ int64_t s_cell[VT];
    const CellLayout& L = p.L;
    const int b = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int D = L.head_dim, G = L.group, R = p.residual;
    const int levels = (1 << L.bits) - 1, pb = 8 / L.bits;
    const int qlen = p.query_start_loc[b + 1] - p.query_start_loc[b];
    const int c = p.seq_lens[b] - qlen;
    if (p.prefilling[b] != 0 || qlen <= 0 || c <= 0) return;

    // ---- keys: whole groups below (c / R) * R, newest first, until a quantized group ----
    for (int s0 = (c / R) * R - G;; s0 -= G) {
        if (tid == 0) {
            const int64_t last = s0 >= 0 ? cell_of(p, b, kvh, s0 + G - 1) : -1;
            s_flag = last < 0 ? 1 : p.cache[last + L.off_flag];
            s_over = 0;
        }
        __syncthreads();
        const int flag = s_flag;
        if (flag != 0) break;
        const int64_t base = cell_of(p, b, kvh, s0);  // a group lies in one page (pages hold whole groups)
        Quant q{};
        if (tid < D) {
            float lo = load_value(p.cache + base, tid, p.format), hi = lo;
            for (int t = 1; t < G; ++t) {
                const float x = load_value(p.cache + base + t * p.sn, tid, p.format);
                lo = __builtin_elementwise_minimum(lo, x);  // NaN propagates, as torch's amin / amax
                hi = __builtin_elementwise_maximum(hi, x);
            }
            q = make_quant(lo, hi, levels, nullptr);
            if (beyond_fp16(q)) atomicOr(&s_over, 1);
            for (int t = 0; t < G; ++t) {
                uint8_t* row = p.cache + base + t * p.sn;
                const uint32_t code = code_of(load_value(row, tid, p.format), q, levels);
                store_value(row, tid, p.format, dequantized(code, q));
                codes[t * D + tid] = static_cast<uint8_t>(code);
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

    // ---- values: tiles of VT tokens below c - R, newest first, while a whole tile was full precision ----
    const int vg = L.value_group, nvg = D / vg;
    for (int top = c - R; top > 0; top -= VT) {
        if (tid < VT) {
            const int t = top - VT + tid;
            const int64_t cell = t >= 0 ? cell_of(p, b, kvh, t) : -1;
            s_cell[tid] = cell;
            s_todo[tid] = cell >= 0 && p.cache[cell + L.off_flag + 1] == 0;
            s_tok_over[tid] = 0;
        }
        __syncthreads();
        for (int item = tid; item < VT * nvg; item += blockDim.x) {
            const int tt = item / nvg, j = item % nvg;
            if (!s_todo[tt]) continue;
            uint8_t* row = p.cache + s_cell[tt] + L.off_v;
            float lo = load_value(row, j * vg, p.format), hi = lo;
            for (int e = 1; e < vg; ++e) {
                const float x = load_value(row, j * vg + e, p.format);
                lo = __builtin_elementwise_minimum(lo, x);
                hi = __builtin_elementwise_maximum(hi, x);
            }
            const Quant q = make_quant(lo, hi, levels, nullptr);
            if (beyond_fp16(q)) atomicOr(&s_tok_over[tt], 1);
            for (int e = 0; e < vg; ++e) {
                const uint32_t code = code_of(load_value(row, j * vg + e, p.format), q, levels);
                store_value(row, j * vg + e, p.format, dequantized(code, q));
                codes[tt * D + j * vg + e] = static_cast<uint8_t>(code);
            }
            store_half(p.cache + s_cell[tt] + L.off_vs + 2 * j, q.scale);
            store_half(p.cache + s_cell[tt] + L.off_vz + 2 * j, q.low);
        }
        __syncthreads();
        const int bytes = D / pb;
        int todo = 0;
        for (int tt = 0; tt < VT; ++tt) todo += s_todo[tt];
        for (int j = tid; j < VT * bytes; j += blockDim.x) {
            const int tt = j / bytes, jj = j % bytes;
            if (!s_todo[tt]) continue;
            uint32_t byte = 0;
            for (int i = 0; i < pb; ++i) byte |= static_cast<uint32_t>(codes[tt * D + jj * pb + i]) << (i * L.bits);
            p.cache[s_cell[tt] + L.off_vc + jj] = static_cast<uint8_t>(byte);
        }
        if (tid < VT && s_todo[tid]) p.cache[s_cell[tid] + L.off_flag + 1] = static_cast<uint8_t>(1 + s_tok_over[tid]);
        __syncthreads();
        if (todo != VT) break;
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

int kivi_cells_quantize(const CellsParams& p, hipStream_t stream) {
    if (p.requests == 0 || p.kv_heads == 0) return 0;
    if (p.L.head_dim > MAX_D || p.L.group > MAX_G)
        return fail("kivi cells: head dims up to 256 and groups up to 128 tokens");
    hipLaunchKernelGGL(kivi_cells_quantize_kernel, dim3(p.requests, p.kv_heads), dim3(256), 0, stream, p);
    return check_launch("kivi_cells_quantize_kernel");
}

int kivi_cells_clear_flags(const CellsParams& p, const int32_t* slots, int tokens, hipStream_t stream) {
    if (tokens == 0) return 0;
    hipLaunchKernelGGL(kivi_cells_clear_kernel, dim3(tokens), dim3(64), 0, stream, p, slots);
    return check_launch("kivi_cells_clear_kernel");
}

}  // namespace eco
