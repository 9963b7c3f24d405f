// KIVI's simulated storage (the reference's KIVICache, techniques/kv_quant/kivi.py:178-275): committed K/V are
// quantized in place inside the dense [B, H, S, D] buffers of the model's dtype. A key group is one channel over
// `group` tokens, a value group `group` channels of one token (the whole head when `group` does not divide it,
// value_group of kivi.py:143-154); every element is replaced by code * scale + low computed in fp32 (the product,
// then the sum: kivi.py:117) and rounded to the buffer's dtype. These are the values the fused kernels dequantize, so
// attention over the buffer is the attention over the codes. Any bits (2, 4, 8) and group size.
//
// Minimum and maximum propagate NaN as torch's amin / amax do, and a NaN code stays NaN, so a group holding NaN
// becomes NaN, as in the reference. One thread per group; O(quantized tokens) bytes, off the decode path.

#include "common.hpp"
#include "kivi_dense.hpp"
#include "kivi_math.hpp"

namespace eco {

namespace {

__device__ inline float load_value(const void* base, int64_t offset, int format) {
    if (format == BF16) return bf16_to_f32(static_cast<const uint16_t*>(base)[offset]);
    if (format == FP16) return static_cast<float>(static_cast<const _Float16*>(base)[offset]);
    return static_cast<const float*>(base)[offset];
}

__device__ inline void store_value(void* base, int64_t offset, int format, float x) {
    if (format == BF16)
        static_cast<uint16_t*>(base)[offset] = f32_to_bf16(x);
    else if (format == FP16)
        static_cast<_Float16*>(base)[offset] = static_cast<_Float16>(x);
    else
        static_cast<float*>(base)[offset] = x;
}

__device__ inline float dequantized(float code, const Quant& q) {
    return __fadd_rn(__fmul_rn(code, q.scale), q.low);  // product then sum, each rounded (no contraction)
}

// Thread per group: keys (b, h, token group, channel), values (b, h, token, channel group). Elements of a group are
// `step` apart in the buffer (the token stride for keys, 1 for values).
__global__ __launch_bounds__(256) void kivi_fake_quant_kernel(KiviFakeParams p) {
    const int levels = (1 << p.bits) - 1;
    const int tokens = p.stop - p.start;
    const int per_row = p.keys ? (tokens / p.group) * p.head_dim : tokens * (p.head_dim / p.group);
    const int64_t total = static_cast<int64_t>(p.batch) * p.heads * per_row;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int item = static_cast<int>(i % per_row);
        const int h = static_cast<int>((i / per_row) % p.heads);
        const int b = static_cast<int>(i / (static_cast<int64_t>(per_row) * p.heads));
        int64_t first, step;
        if (p.keys) {
            const int tg = item / p.head_dim, d = item % p.head_dim;
            first = b * p.sb + h * p.sh + static_cast<int64_t>(p.start + tg * p.group) * p.ss + d;
            step = p.ss;
        } else {
            const int t = item / (p.head_dim / p.group), g = item % (p.head_dim / p.group);
            first = b * p.sb + h * p.sh + static_cast<int64_t>(p.start + t) * p.ss + g * p.group;
            step = 1;
        }
        float lo = load_value(p.buf, first, p.format), hi = lo;
        for (int e = 1; e < p.group; ++e) {
            const float x = load_value(p.buf, first + e * step, p.format);
            lo = __builtin_elementwise_minimum(lo, x);
            hi = __builtin_elementwise_maximum(hi, x);
        }
        const Quant q = make_quant(lo, hi, levels, nullptr);
        for (int e = 0; e < p.group; ++e) {
            const float x = load_value(p.buf, first + e * step, p.format);
            store_value(p.buf, first + e * step, p.format, dequantized(code_or_nan(x, q, levels), q));
        }
    }
}

__device__ inline uint16_t half_bits(float x) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x)); }

// Keys into the packed record: a thread per (b, h, key group after from[b], code byte j), the 8 / bits channels of
// byte j over the group's tokens (their quantization first, then the tokens' code bytes), so that no two threads
// write one byte.
__global__ __launch_bounds__(256) void kivi_pack_keys_kernel(KiviPackParams p) {
    const int levels = (1 << p.bits) - 1;
    const int per_byte = 8 / p.bits;
    const int bytes = p.head_dim / per_byte;
    const int groups = p.max_tokens / p.group;
    const int64_t total = static_cast<int64_t>(p.batch) * p.heads * groups * bytes;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int j = static_cast<int>(i % bytes);
        const int gi = static_cast<int>((i / bytes) % groups);
        const int h = static_cast<int>((i / (static_cast<int64_t>(bytes) * groups)) % p.heads);
        const int b = static_cast<int>(i / (static_cast<int64_t>(bytes) * groups * p.heads));
        const int s0 = p.from[b] + gi * p.group;
        if (s0 < 0 || s0 + p.group > min(p.to[b], p.slots)) continue;
        const int64_t base = b * p.ss_b + h * p.ss_h;
        auto at = [&](int s, int d) {
            const int slot = p.src_ring > 0 ? s % p.src_ring : s;
            return base + static_cast<int64_t>(slot) * p.ss_s + d;
        };
        Quant q[4];
        for (int c = 0; c < per_byte; ++c) {
            const int d = j * per_byte + c;
            float lo = load_value(p.src, at(s0, d), p.format), hi = lo;
            for (int e = 1; e < p.group; ++e) {
                const float x = load_value(p.src, at(s0 + e, d), p.format);
                lo = __builtin_elementwise_minimum(lo, x);
                hi = __builtin_elementwise_maximum(hi, x);
            }
            q[c] = make_quant(lo, hi, levels, p.overflow);
            const int64_t so = b * p.sz_b + h * p.sz_h + static_cast<int64_t>(s0 / p.group) * p.sz_s + d;
            p.scale[so] = half_bits(q[c].scale);
            p.zero[so] = half_bits(q[c].low);
        }
        uint8_t* crow = p.codes + b * p.sc_b + h * p.sc_h + j;
        for (int e = 0; e < p.group; ++e) {
            uint32_t byte = 0;
            for (int c = 0; c < per_byte; ++c) {
                const int64_t o = at(s0 + e, j * per_byte + c);
                const float x = load_value(p.src, o, p.format);
                byte |= code_of(x, q[c], levels) << (c * p.bits);
                if (p.write_back) store_value(p.src, o, p.format, dequantized(code_or_nan(x, q[c], levels), q[c]));
            }
            crow[static_cast<int64_t>(s0 + e) * p.sc_s] = static_cast<uint8_t>(byte);
        }
    }
}

// Values into the packed record: a thread per (b, h, token after from[b]), its groups in order, the code bytes
// assembled across group boundaries.
__global__ __launch_bounds__(256) void kivi_pack_values_kernel(KiviPackParams p) {
    const int levels = (1 << p.bits) - 1;
    const int per_byte = 8 / p.bits;
    const int64_t total = static_cast<int64_t>(p.batch) * p.heads * p.max_tokens;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int ti = static_cast<int>(i % p.max_tokens);
        const int h = static_cast<int>((i / p.max_tokens) % p.heads);
        const int b = static_cast<int>(i / (static_cast<int64_t>(p.max_tokens) * p.heads));
        const int s = p.from[b] + ti;
        if (s < 0 || s >= min(p.to[b], p.slots)) continue;
        const int slot = p.src_ring > 0 ? s % p.src_ring : s;
        const int64_t row = b * p.ss_b + h * p.ss_h + static_cast<int64_t>(slot) * p.ss_s;
        uint8_t* crow = p.codes + b * p.sc_b + h * p.sc_h + static_cast<int64_t>(s) * p.sc_s;
        const int64_t srow = b * p.sz_b + h * p.sz_h + static_cast<int64_t>(s) * p.sz_s;
        uint32_t byte = 0;
        for (int g0 = 0; g0 < p.head_dim; g0 += p.group) {
            float lo = load_value(p.src, row + g0, p.format), hi = lo;
            for (int e = 1; e < p.group; ++e) {
                const float x = load_value(p.src, row + g0 + e, p.format);
                lo = __builtin_elementwise_minimum(lo, x);
                hi = __builtin_elementwise_maximum(hi, x);
            }
            const Quant q = make_quant(lo, hi, levels, p.overflow);
            p.scale[srow + g0 / p.group] = half_bits(q.scale);
            p.zero[srow + g0 / p.group] = half_bits(q.low);
            for (int e = 0; e < p.group; ++e) {
                const int d = g0 + e;
                const float x = load_value(p.src, row + d, p.format);
                byte |= code_of(x, q, levels) << ((d % per_byte) * p.bits);
                if (d % per_byte == per_byte - 1) {
                    crow[d / per_byte] = static_cast<uint8_t>(byte);
                    byte = 0;
                }
                if (p.write_back) store_value(p.src, row + d, p.format, dequantized(code_or_nan(x, q, levels), q));
            }
        }
    }
}

// A thread per output element: its code and its group's scale and zero point, or its ring entry.
__global__ __launch_bounds__(256) void kivi_packed_gather_kernel(KiviRecordGatherParams p) {
    const int per_byte = 8 / p.bits;
    const int64_t total = static_cast<int64_t>(p.batch) * p.heads * p.slots * p.head_dim;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int d = static_cast<int>(i % p.head_dim);
        const int s = static_cast<int>((i / p.head_dim) % p.slots);
        const int h = static_cast<int>((i / (static_cast<int64_t>(p.head_dim) * p.slots)) % p.heads);
        const int b = static_cast<int>(i / (static_cast<int64_t>(p.head_dim) * p.slots * p.heads));
        float x;
        if (s < p.quantized[b]) {
            const uint32_t byte = p.codes[b * p.sc_b + h * p.sc_h + static_cast<int64_t>(s) * p.sc_s + d / per_byte];
            const float code = static_cast<float>((byte >> ((d % per_byte) * p.bits)) & ((1u << p.bits) - 1u));
            const int64_t so = b * p.sz_b + h * p.sz_h +
                               (p.keys ? static_cast<int64_t>(s / p.group) * p.sz_s + d
                                       : static_cast<int64_t>(s) * p.sz_s + d / p.group);
            const float sc = static_cast<float>(__builtin_bit_cast(_Float16, p.scale[so]));
            const float zr = static_cast<float>(__builtin_bit_cast(_Float16, p.zero[so]));
            x = __fadd_rn(__fmul_rn(code, sc), zr);
        } else {
            const int slot = p.ring_slots > 0 ? s % p.ring_slots : s;
            x = load_value(p.ring, b * p.sr_b + h * p.sr_h + static_cast<int64_t>(slot) * p.sr_s + d, p.format);
        }
        store_value(p.out, b * p.so_b + h * p.so_h + static_cast<int64_t>(s) * p.so_s + d, p.format, x);
    }
}

}  // namespace

int kivi_packed_gather(const KiviRecordGatherParams& p, hipStream_t stream) {
    const int64_t items = static_cast<int64_t>(p.batch) * p.heads * p.slots * p.head_dim;
    if (items == 0) return 0;
    const int blocks = static_cast<int>((items + 255) / 256 < 65535 ? (items + 255) / 256 : 65535);
    hipLaunchKernelGGL(kivi_packed_gather_kernel, dim3(blocks), dim3(256), 0, stream, p);
    return check_launch("kivi_packed_gather_kernel");
}

int kivi_pack_quantize(const KiviPackParams& p, hipStream_t stream) {
    const int64_t items = static_cast<int64_t>(p.batch) * p.heads *
                          (p.keys ? (p.max_tokens / p.group) * (p.head_dim * p.bits / 8) : p.max_tokens);
    if (items == 0) return 0;
    const int blocks = static_cast<int>((items + 255) / 256 < 65535 ? (items + 255) / 256 : 65535);
    if (p.keys)
        hipLaunchKernelGGL(kivi_pack_keys_kernel, dim3(blocks), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(kivi_pack_values_kernel, dim3(blocks), dim3(256), 0, stream, p);
    return check_launch(p.keys ? "kivi_pack_keys_kernel" : "kivi_pack_values_kernel");
}

int kivi_fake_quantize(const KiviFakeParams& p, hipStream_t stream) {
    const int tokens = p.stop - p.start;
    const int64_t groups = static_cast<int64_t>(p.batch) * p.heads *
                           (p.keys ? (tokens / p.group) * p.head_dim : tokens * (p.head_dim / p.group));
    if (groups == 0) return 0;
    const int blocks = static_cast<int>((groups + 255) / 256 < 65535 ? (groups + 255) / 256 : 65535);
    hipLaunchKernelGGL(kivi_fake_quant_kernel, dim3(blocks), dim3(256), 0, stream, p);
    return check_launch("kivi_fake_quant_kernel");
}

}  // namespace eco
