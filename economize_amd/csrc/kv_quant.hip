// FP8 / bf16 quantize-and-append into the paged KV cache, and per-head absmax scales (gfx950).
//
// Append follows the reference's fp8 encode (techniques/kv_quant/fp8.py:81-86, FP8Cache.transform_update
// fp8.py:161-176): x.float() / scale with IEEE division, clamp to the format's finite maximum, cast with
// round-to-nearest-even (f32_to_fp8 in common.hpp), written at the token's slot (vLLM-style slot mapping: slot =
// page * 16 + position; a negative slot is padding and writes nothing, like the trash slot of
// modules/kv_cache.py:13-27). The per-head scale is the reference's static_scales rule (fp8.py:130-133) over each
// KV head's absolute maximum.
//
// Layout of the caches: see paged_attention.hip. One workgroup per new token; a thread encodes 8 consecutive
// channels of one head, so the key write is one 8-byte (fp8) or 16-byte (bf16) store into the token's 16-byte run,
// and the value write scatters the 8 channels into their channel rows.

#include "common.hpp"
#include "kv_quant.hpp"
#include "quest_page.hpp"

namespace eco {

namespace {

constexpr int PAGE = 16;

__device__ inline float load_elem(const void* base, int64_t offset, int format) {
    if (format == BF16) return bf16_to_f32(static_cast<const uint16_t*>(base)[offset]);
    if (format == FP16) return static_cast<float>(static_cast<const _Float16*>(base)[offset]);
    return static_cast<const float*>(base)[offset];
}

template <int FMT>
__device__ inline uint8_t encode(float x, float scale, bool scaled) {
    float w = scaled ? __fdiv_rn(x, scale) : x;
    if (w != w) return f32_to_fp8<FMT>(x != x ? x : w);  // NaN stays NaN (fminf/fmaxf would drop it)
    return f32_to_fp8<FMT>(fminf(fmaxf(w, -fp8_max<FMT>()), fp8_max<FMT>()));
}

// New token t into its slot, by one workgroup.
template <int FMT>
__device__ inline void append_token(const AppendParams& p, int t) {
    constexpr int ES = FMT == BF16 ? 2 : 1;
    constexpr int E = 16 / ES;  // channels per 16-byte run of the key layout
    const int slot = p.slots[t];
    if (slot < 0 || slot / PAGE >= p.num_pages) return;
    const int page = slot / PAGE;
    const int pos = slot % PAGE;
    const int runs = p.head_dim / 8;
    for (int item = threadIdx.x; item < p.kv_heads * runs; item += blockDim.x) {
        const int h = item / runs;
        const int d0 = (item % runs) * 8;
        const float ks = p.k_scale ? p.k_scale[h] : 1.0f;
        const float vs = p.v_scale ? p.v_scale[h] : 1.0f;
        float k[8], v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            k[i] = load_elem(p.k_new, t * p.sk_t + h * p.sk_h + d0 + i, p.in_format);
            v[i] = load_elem(p.v_new, t * p.sv_t + h * p.sv_h + d0 + i, p.in_format);
        }
        uint8_t* kp = p.k_cache + static_cast<int64_t>(page) * p.kc_page + h * p.kc_head;
        uint8_t* vp = p.v_cache + static_cast<int64_t>(page) * p.vc_page + h * p.vc_head;
        const int64_t k_off = ((d0 / E) * PAGE + pos) * 16 + (d0 % E) * ES;
        if constexpr (FMT == BF16) {
            uint4 w;
            w.x = f32_to_bf16(k[0]) | (static_cast<uint32_t>(f32_to_bf16(k[1])) << 16);
            w.y = f32_to_bf16(k[2]) | (static_cast<uint32_t>(f32_to_bf16(k[3])) << 16);
            w.z = f32_to_bf16(k[4]) | (static_cast<uint32_t>(f32_to_bf16(k[5])) << 16);
            w.w = f32_to_bf16(k[6]) | (static_cast<uint32_t>(f32_to_bf16(k[7])) << 16);
            *reinterpret_cast<uint4*>(kp + k_off) = w;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                *reinterpret_cast<uint16_t*>(vp + ((d0 + i) * PAGE + pos) * 2) = f32_to_bf16(v[i]);
        } else {
            const bool scaled = p.k_scale != nullptr;
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo |= static_cast<uint32_t>(encode<FMT>(k[i], ks, scaled)) << (8 * i);
                hi |= static_cast<uint32_t>(encode<FMT>(k[i + 4], ks, scaled)) << (8 * i);
            }
            *reinterpret_cast<uint2*>(kp + k_off) = make_uint2(lo, hi);
            const bool vscaled = p.v_scale != nullptr;
#pragma unroll
            for (int i = 0; i < 8; ++i) vp[(d0 + i) * PAGE + pos] = encode<FMT>(v[i], vs, vscaled);
        }
    }
}

template <int FMT>
__global__ __launch_bounds__(256) void paged_append_kernel(AppendParams p) {
    append_token<FMT>(p, blockIdx.x);
}

// The append with Quest's metadata kept on the device, in one launch: workgroups below `tokens` append a token each;
// the others are four waves each of the refresh, kRefreshWaves waves per (row, KV head) taking the Quest pages
// valid + y, valid + y + kRefreshWaves, ... below the row's committed pages (the bounds of pages that became committed,
// quest_refresh_kernel's work). The last of a row's waves to finish (a counter per row, agent-scope atomics; every
// wave has read valid before it counts itself) advances valid and writes done, then leaves the counter zero. The
// tokens appended lie at or past the committed ones, so no page this launch refreshes is written by it.
constexpr int kRefreshWaves = 8;

template <int FMT>
__global__ __launch_bounds__(256) void paged_append_quest_kernel(AppendParams p, BoundsParams q, int32_t* counters) {
    if (static_cast<int>(blockIdx.x) < p.tokens) {
        append_token<FMT>(p, blockIdx.x);
        return;
    }
    const int wave = (static_cast<int>(blockIdx.x) - p.tokens) * 4 + static_cast<int>(threadIdx.x >> 6);
    const int lane = static_cast<int>(threadIdx.x & 63);
    if (wave >= q.batch * q.kv_heads * kRefreshWaves) return;
    const int row = wave / kRefreshWaves, y = wave % kRefreshWaves;
    const int b = row / q.kv_heads, kvh = row % q.kv_heads;
    const int last = min(max(q.committed[b], 0) / (16 * q.span), q.page_cap);
    const int from = q.valid[row];
    for (int qp = from + y; qp < last; qp += kRefreshWaves) quest_bounds_of_page<FMT>(q, b, qp, kvh, lane);
    int prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(counters + row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__shfl(prev, 0) != kRefreshWaves - 1) return;
    if (lane == 0) {
        q.valid[row] = max(from, last);
        if (q.done && kvh == 0) q.done[b] = last;
        __hip_atomic_store(counters + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Dense encode (fp8_encode of fp8.py:81-86 over a [B, H, T, D] block, the fused fp8 cache's dense buffers of
// kv_fp8_fused/fused.py:56-63): one wave per (b, h, t) row, each lane a few channels. The per-token mode computes the
// row's scale as token_scale does (fp8.py:95-97: absmax / format max with IEEE division, at least 1e-12), writes it
// and encodes with it; the per-head mode divides by head_scale[h]; with neither the values are cast directly.
template <int FMT>
__global__ __launch_bounds__(256) void fp8_encode_kernel(EncodeParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t rows = static_cast<int64_t>(p.batch) * p.heads * p.tokens;
    for (int64_t row = blockIdx.x * 4LL + (threadIdx.x >> 6); row < rows; row += static_cast<int64_t>(gridDim.x) * 4) {
        const int t = static_cast<int>(row % p.tokens);
        const int h = static_cast<int>((row / p.tokens) % p.heads);
        const int b = static_cast<int>(row / (static_cast<int64_t>(p.tokens) * p.heads));
        const int64_t src = b * p.ss_b + h * p.ss_h + t * p.ss_t;
        uint8_t* dst = p.dst + b * p.sd_b + h * p.sd_h + t * p.sd_t;
        float x[8];  // channels lane, lane + 64, .. (head dims up to 512)
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int d = lane + 64 * i;
            x[i] = d < p.head_dim ? load_elem(p.src, src + d, p.in_format) : 0.0f;
            amax = fmaxf(amax, fabsf(x[i]));
        }
        float scale = 1.0f;
        bool scaled = false;
        if (p.token_scale) {
            bool nan = false;  // torch's amax propagates NaN, and so does the scale then
#pragma unroll
            for (int i = 0; i < 8; ++i) nan |= x[i] != x[i];
            for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
            scale = __ballot(nan) ? __builtin_nanf("") : fmaxf(__fdiv_rn(amax, fp8_max<FMT>()), 1e-12f);
            scaled = true;
            if (lane == 0) p.token_scale[b * p.st_b + h * p.st_h + t * p.st_t] = scale;
        } else if (p.head_scale) {
            scale = p.head_scale[h];
            scaled = true;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int d = lane + 64 * i;
            if (d < p.head_dim) dst[d] = encode<FMT>(x[i], scale, scaled);
        }
    }
}

// absmax[h] = max |x[a, h, s, d]| as float bits (non-negative floats order like their bit patterns).
__global__ __launch_bounds__(256) void head_absmax_kernel(AbsmaxParams p) {
    const int h = blockIdx.y;
    const int64_t total = static_cast<int64_t>(p.a) * p.s * p.d;
    float m = 0.0f;
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t a = idx / (static_cast<int64_t>(p.s) * p.d);
        const int64_t s = (idx / p.d) % p.s;
        const int64_t d = idx % p.d;
        const float x = load_elem(p.x, a * p.sa + h * p.sh + s * p.ss + d * p.sd, p.in_format);
        m = fmaxf(m, fabsf(x));
    }
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) atomicMax(p.absmax_bits + h, f32_bits(m));
}

// static_scales (fp8.py:130-133): absmax / format max with IEEE division, 1 where that is not positive.
__global__ void scales_from_absmax_kernel(const uint32_t* absmax_bits, int heads, float format_max, float* scales) {
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h < heads) {
        const float s = __fdiv_rn(bits_f32(absmax_bits[h]), format_max);
        scales[h] = s > 0.0f ? s : 1.0f;
    }
}

}  // namespace

int paged_append(const AppendParams& p, hipStream_t stream) {
    if (p.tokens == 0) return 0;
    dim3 grid(p.tokens);
    switch (p.cache_format) {
        case BF16: hipLaunchKernelGGL(paged_append_kernel<BF16>, grid, dim3(256), 0, stream, p); break;
        case FP8_E4M3: hipLaunchKernelGGL(paged_append_kernel<FP8_E4M3>, grid, dim3(256), 0, stream, p); break;
        case FP8_E5M2: hipLaunchKernelGGL(paged_append_kernel<FP8_E5M2>, grid, dim3(256), 0, stream, p); break;
        default: return fail("paged append: cache format must be bf16, fp8 e4m3 or fp8 e5m2");
    }
    return check_launch("paged_append_kernel");
}

int paged_append_quest(const AppendParams& p, const BoundsParams& q, int32_t* counters, hipStream_t stream) {
    const int refresh = (q.batch * q.kv_heads * kRefreshWaves + 3) / 4;
    dim3 grid(p.tokens + refresh);
    switch (p.cache_format) {
        case BF16: hipLaunchKernelGGL(paged_append_quest_kernel<BF16>, grid, dim3(256), 0, stream, p, q, counters); break;
        case FP8_E4M3:
            hipLaunchKernelGGL(paged_append_quest_kernel<FP8_E4M3>, grid, dim3(256), 0, stream, p, q, counters);
            break;
        case FP8_E5M2:
            hipLaunchKernelGGL(paged_append_quest_kernel<FP8_E5M2>, grid, dim3(256), 0, stream, p, q, counters);
            break;
        default: return fail("paged append: cache format must be bf16, fp8 e4m3 or fp8 e5m2");
    }
    return check_launch("paged_append_quest_kernel");
}

int fp8_encode(const EncodeParams& p, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(p.batch) * p.heads * p.tokens;
    if (rows == 0) return 0;
    const int blocks = static_cast<int>((rows + 3) / 4 < 65535 ? (rows + 3) / 4 : 65535);
    switch (p.out_format) {
        case FP8_E4M3: hipLaunchKernelGGL(fp8_encode_kernel<FP8_E4M3>, dim3(blocks), dim3(256), 0, stream, p); break;
        case FP8_E5M2: hipLaunchKernelGGL(fp8_encode_kernel<FP8_E5M2>, dim3(blocks), dim3(256), 0, stream, p); break;
        default: return fail("fp8 encode: the output format must be fp8 e4m3 or e5m2");
    }
    return check_launch("fp8_encode_kernel");
}

int head_absmax(const AbsmaxParams& p, hipStream_t stream) {
    const int64_t total = static_cast<int64_t>(p.a) * p.s * p.d;
    int blocks = static_cast<int>((total + 256 * 16 - 1) / (256 * 16));
    blocks = blocks < 1 ? 1 : (blocks > 1024 ? 1024 : blocks);
    hipLaunchKernelGGL(head_absmax_kernel, dim3(blocks, p.h), dim3(256), 0, stream, p);
    return check_launch("head_absmax_kernel");
}

int scales_from_absmax(const uint32_t* absmax_bits, int heads, int format, float* scales, hipStream_t stream) {
    const float fmax = format == FP8_E4M3 ? 448.0f : 57344.0f;
    hipLaunchKernelGGL(scales_from_absmax_kernel, dim3((heads + 63) / 64), dim3(64), 0, stream, absmax_bits, heads,
                       fmax, scales);
    return check_launch("scales_from_absmax_kernel");
}

}  // namespace eco
