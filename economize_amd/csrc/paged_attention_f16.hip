// The launches of the paged decode-attention kernel (paged_kernel.hpp) with fp16 queries and output over an fp8 cache
// (a model in fp16 with its cache in fp8): the keys are converted to fp16, exactly, for the fp16 MFMA. The instances
// are those the bf16-query dispatch uses by default (two tile buffers where they fit, streamed loads of whole rows);
// Quest's page lists read a bf16 cache and keep bf16 queries.

#include "paged_kernel.hpp"

namespace eco {

namespace {

using KernelFnH = decltype(&paged_attention_kernel<64, FP8_E4M3, 1, 1, true, true>);
struct InstanceH {
    KernelFnH kernel;
    int waves;
};

template <int D, int FMT, int NB>
InstanceH instance_f16() {
    constexpr int S = D <= 128 && NB <= 2 ? 2 : 1;  // tile buffers
    return {paged_attention_kernel<D, FMT, NB, S, true, true>, wg_waves<D, FMT, NB, S>()};
}

template <typename F>
int dispatch_f16(int head_dim, int format, int rows, const F& f) {
    const int nb = (rows + 15) / 16;
    auto by_nb = [&](auto d_tag, auto fmt_tag) __attribute__((always_inline)) -> int {
        constexpr int D = decltype(d_tag)::value;
        constexpr int FMT = decltype(fmt_tag)::value;
        if (nb == 1) return f(instance_f16<D, FMT, 1>());
        if (nb == 2) return f(instance_f16<D, FMT, 2>());
        if (nb <= 4) return f(instance_f16<D, FMT, 4>());
        return fail("paged decode attention takes at most 64 query rows per KV head (query heads per KV head x "
                    "queries)");
    };
    auto by_fmt = [&](auto d_tag) __attribute__((always_inline)) -> int {
        switch (format) {
            case FP8_E4M3: return by_nb(d_tag, std::integral_constant<int, FP8_E4M3>{});
            case FP8_E5M2: return by_nb(d_tag, std::integral_constant<int, FP8_E5M2>{});
            default: return fail("paged decode: fp16 queries read an fp8 e4m3 or e5m2 cache");
        }
    };
    switch (head_dim) {
        case 64: return by_fmt(std::integral_constant<int, 64>{});
        case 128: return by_fmt(std::integral_constant<int, 128>{});
        case 256: return by_fmt(std::integral_constant<int, 256>{});
        default: return fail("paged decode attention supports head dims 64, 128 and 256");
    }
}

}  // namespace

int paged_resident_groups_f16(int head_dim, int format, int rows, int* per_cu, int* waves) {
    return dispatch_f16(head_dim, format, rows, [&](const InstanceH& in) {
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, in.kernel, 64 * in.waves, 0) != hipSuccess ||
            blocks <= 0)
            blocks = 1;
        *per_cu = blocks;
        *waves = in.waves;
        return 0;
    });
}

int paged_attention_f16(const PagedParams& p, hipStream_t stream) {
    if (p.page_list) return fail("paged decode: page lists take bf16 queries");
    return dispatch_f16(p.head_dim, p.kv_format, p.rows, [&](const InstanceH& in) {
        hipLaunchKernelGGL(in.kernel, dim3(p.grid), dim3(64 * in.waves), 0, stream, p);
        return check_launch("paged_attention_kernel (fp16 queries)");
    });
}

}  // namespace eco
