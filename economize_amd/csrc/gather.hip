// Dense views of the paged caches (the reference's materialize(), attention/packed.py:66-78): the K/V that the
// attention kernels read, written out as [B, Hkv, S, D] for the attention functions that do not read the paged
// formats (a long prompt's attention, the fallbacks). Elementwise and HBM-bound: one 16-byte group of eight channels
// per thread.

#include "common.hpp"
#include "gather.hpp"
#include "kivi.hpp"

namespace eco {

namespace {

__device__ inline void store_elem(void* base, int64_t offset, int format, float x) {
    if (format == BF16)
        static_cast<uint16_t*>(base)[offset] = f32_to_bf16(x);
    else if (format == FP16)
        static_cast<_Float16*>(base)[offset] = static_cast<_Float16>(x);
    else
        static_cast<float*>(base)[offset] = x;
}

__device__ inline float cache_elem(const uint8_t* p, int format) {
    if (format == BF16) return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const uint32_t w = *p;
    const f32x2 r = format == FP8_E4M3 ? __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false)
                                       : __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(w, 1.0f, false);
    return r.x;
}

// thread i: row b, head h, token t, channels 8 c .. 8 c + 7 (t < keys; tokens past a row's table read nothing and
// give 0).
__global__ __launch_bounds__(256) void paged_gather_kernel(PagedGatherParams p) {
    const int groups = p.head_dim / 8;
    const int64_t total = static_cast<int64_t>(p.batch) * p.kv_heads * p.keys * groups;
    const int es = p.kv_format == BF16 ? 2 : 1;
    const int x = 16 / es;  // channels per 16-byte key run
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int c = static_cast<int>(i % groups);
        const int t = static_cast<int>((i / groups) % p.keys);
        const int h = static_cast<int>((i / (static_cast<int64_t>(groups) * p.keys)) % p.kv_heads);
        const int b = static_cast<int>(i / (static_cast<int64_t>(groups) * p.keys * p.kv_heads));
        const int lp = t / 16, pos = t % 16;
        int page = lp < p.bt_cols ? p.block_table[b * p.bt_stride + lp] : -1;
        page = page < p.num_pages ? page : -1;
        const float ks = p.k_scale ? p.k_scale[h] : 1.0f;
        const float vs = p.v_scale ? p.v_scale[h] : 1.0f;
        const int64_t ko = b * p.so_kb + h * p.so_kh + t * p.so_ks + 8 * c;
        const int64_t vo = b * p.so_vb + h * p.so_vh + t * p.so_vs + 8 * c;
        for (int e = 0; e < 8; ++e) {
            const int d = 8 * c + e;
            float kx = 0.0f, vx = 0.0f;
            if (page >= 0) {
                const uint8_t* kp = p.k_cache + (page * p.kc_page + h * p.kc_head) +
                                    ((static_cast<int64_t>(d / x) * 16 + pos) * x + d % x) * es;
                const uint8_t* vp = p.v_cache + (page * p.vc_page + h * p.vc_head) +
                                    (static_cast<int64_t>(d) * 16 + pos) * es;
                kx = cache_elem(kp, p.kv_format) * ks;
                vx = cache_elem(vp, p.kv_format) * vs;
            }
            store_elem(p.k_out, ko + e, p.out_format, kx);
            store_elem(p.v_out, vo + e, p.out_format, vx);
        }
    }
}

// The code of element e of a 32-bit word of 32 / bits elements: byte e % 4, bit (e / 4) * bits.
__device__ inline uint32_t code_at(const uint8_t* words, int e, int bits) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(words)[e / (32 / bits)];
    const int k = e % (32 / bits);
    return (w >> (8 * (k % 4) + (k / 4) * bits)) & ((1u << bits) - 1);
}

__device__ inline float half_at(const uint8_t* p, int index) {
    return static_cast<float>(reinterpret_cast<const _Float16*>(p)[index]);
}

// thread i: row b, head h, token t, channels 8 c .. 8 c + 7: keys below keys_quantized[b] and values below
// values_quantized[b] dequantized as the reference's dequantize (bf16(code * scale + zero), product and sum in fp32),
// the others from the rings.
__global__ __launch_bounds__(256) void kivi_gather_kernel(KiviGatherParams p) {
    const int d_all = p.head_dim;
    const int groups = d_all / 8;
    const KiviLayout L{p.head_dim, p.bits};
    const int64_t total = static_cast<int64_t>(p.batch) * p.kv_heads * p.keys * groups;
    const int tpw = 32 / p.bits;
    const int nd_count = p.head_dim / 16;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int c = static_cast<int>(i % groups);
        const int t = static_cast<int>((i / groups) % p.keys);
        const int h = static_cast<int>((i / (static_cast<int64_t>(groups) * p.keys)) % p.kv_heads);
        const int b = static_cast<int>(i / (static_cast<int64_t>(groups) * p.keys * p.kv_heads));
        const int kq = p.keys_quantized[b], vq = p.values_quantized[b];
        const int lp = t / 32, pos = t % 32;
        int page = lp < p.bt_cols ? p.block_table[b * p.bt_stride + lp] : -1;
        page = page < p.num_pages ? page : -1;
        const uint8_t* blk = page >= 0 ? p.blocks + (page * p.blk_page + h * p.blk_head) : nullptr;
        const int64_t row = static_cast<int64_t>(b) * p.kv_heads + h;
        const int slot = t % p.ring;
        const int64_t ko = b * p.so_kb + h * p.so_kh + t * p.so_ks + 8 * c;
        const int64_t vo = b * p.so_vb + h * p.so_vh + t * p.so_vs + 8 * c;
        for (int e = 0; e < 8; ++e) {
            const int d = 8 * c + e;
            float kx = 0.0f, vx = 0.0f;
            if (t < kq) {
                if (blk) {
                    const uint32_t code = code_at(blk + L.k_codes() + pos * (p.head_dim * p.bits / 8), d, p.bits);
                    kx = bf16_to_f32(f32_to_bf16(__builtin_fmaf(static_cast<float>(code), half_at(blk + L.k_scale(), d),
                                                                half_at(blk + L.k_zero(), d))));
                }
            } else {
                kx = bf16_to_f32(p.k_ring[(row * p.ring + slot) * p.head_dim + d]);
            }
            if (t < vq) {
                if (blk) {
                    const int u = pos / tpw, nd = d / 16, n = d % 16;
                    const uint8_t* word = blk + L.v_codes() + 4 * ((u * 16 + n) * nd_count + nd);
                    const uint32_t code = code_at(word, pos % tpw, p.bits);
                    const int grp = d / 32;
                    vx = bf16_to_f32(f32_to_bf16(__builtin_fmaf(static_cast<float>(code),
                                                                half_at(blk + L.v_scale(), grp * 32 + pos),
                                                                half_at(blk + L.v_zero(), grp * 32 + pos))));
                }
            } else {
                vx = bf16_to_f32(p.v_ring[(row * p.head_dim + d) * p.ring + slot]);
            }
            store_elem(p.k_out, ko + e, p.out_format, kx);
            store_elem(p.v_out, vo + e, p.out_format, vx);
        }
    }
}

int grid_of(int64_t total) { return static_cast<int>(total / 256 + 1 < 65535 ? total / 256 + 1 : 65535); }

}  // namespace

int paged_gather(const PagedGatherParams& p, hipStream_t stream) {
    const int64_t total = static_cast<int64_t>(p.batch) * p.kv_heads * p.keys * (p.head_dim / 8);
    if (total == 0) return 0;
    hipLaunchKernelGGL(paged_gather_kernel, dim3(grid_of(total)), dim3(256), 0, stream, p);
    return check_launch("paged_gather_kernel");
}

int kivi_gather(const KiviGatherParams& p, hipStream_t stream) {
    const int64_t total = static_cast<int64_t>(p.batch) * p.kv_heads * p.keys * (p.head_dim / 8);
    if (total == 0) return 0;
    hipLaunchKernelGGL(kivi_gather_kernel, dim3(grid_of(total)), dim3(256), 0, stream, p);
    return check_launch("kivi_gather_kernel");
}

}  // namespace eco
