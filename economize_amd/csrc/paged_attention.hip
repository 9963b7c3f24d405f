// The launches of the paged decode-attention kernel (paged_kernel.hpp) with bf16 queries: the instance for the head
// dim, the KV format, the query rows and the tile buffers; fp16 queries go to paged_attention_f16.hip.

#include "paged_kernel.hpp"

namespace eco {

// ---- host side ----------------------------------------------------------------------------------------------

namespace {

// Tile buffers of an instance: two where they fit in the registers beside the accumulators (a tile of fp8 K/V at
// D = 128 is 64 VGPRs per lane, plus 16 of query operand). Three fit for one column block, but measured slower at
// the Llama-3-8B decode shape (55.0 against 53.6 us; ragged lengths 77.1 against 71.8 us). ECO_PAGED_STAGES (1 to 3)
// selects the count for tuning.
template <int D, int FMT, int NB>
constexpr int max_stages() {
    if (FMT != BF16 && D <= 128 && NB == 1) return 3;
    if (FMT != BF16 && D <= 128 && NB == 2) return 2;
    return 1;
}

int stages_cap() {
    static const int cap = [] {
        const char* env = std::getenv("ECO_PAGED_STAGES");
        const int v = env ? std::atoi(env) : 2;
        return v < 1 ? 1 : (v > 3 ? 3 : v);
    }();
    return cap;
}

// The kernel instance for the tile-buffer count, and its waves per workgroup.
using KernelFn = decltype(&paged_attention_kernel<64, BF16, 1, 1, false>);
struct Instance {
    KernelFn kernel;
    int waves;
};

template <int D, int FMT, int NB, bool NT>
Instance kernel_of() {
    constexpr int M = max_stages<D, FMT, NB>();
    const int s = stages_cap() < M ? stages_cap() : M;
    if constexpr (M >= 3)
        if (s == 3) return {paged_attention_kernel<D, FMT, NB, 3, NT>, wg_waves<D, FMT, NB, 3>()};
    if constexpr (M >= 2)
        if (s >= 2) return {paged_attention_kernel<D, FMT, NB, 2, NT>, wg_waves<D, FMT, NB, 2>()};
    return {paged_attention_kernel<D, FMT, NB, 1, NT>, wg_waves<D, FMT, NB, 1>()};
}

// Streamed tile loads for calls that read whole rows; plain ones for page lists (see load16).
template <int D, int FMT, int NB>
Instance kernel_of(bool page_list) {
    return page_list ? kernel_of<D, FMT, NB, false>() : kernel_of<D, FMT, NB, true>();
}

// Calls f.template run<D, FMT, NB>() for the instance of (head dim, format, 16-row column blocks).
template <typename F>
int dispatch(int head_dim, int format, int rows, const F& f) {
    const int nb = (rows + 15) / 16;
    auto by_nb = [&](auto d_tag, auto fmt_tag) __attribute__((always_inline)) -> int {
        constexpr int D = decltype(d_tag)::value;
        constexpr int FMT = decltype(fmt_tag)::value;
        if (nb == 1) return f.template run<D, FMT, 1>();
        if (nb == 2) return f.template run<D, FMT, 2>();
        if (nb <= 4) return f.template run<D, FMT, 4>();
        return fail("paged decode attention takes at most 64 query rows per KV head (query heads per KV head x "
                    "queries)");
    };
    auto by_fmt = [&](auto d_tag) __attribute__((always_inline)) -> int {
        switch (format) {
            case BF16: return by_nb(d_tag, std::integral_constant<int, BF16>{});
            case FP8_E4M3: return by_nb(d_tag, std::integral_constant<int, FP8_E4M3>{});
            case FP8_E5M2: return by_nb(d_tag, std::integral_constant<int, FP8_E5M2>{});
            default: return fail("paged decode attention: KV format must be bf16, fp8 e4m3 or fp8 e5m2");
        }
    };
    switch (head_dim) {
        case 64: return by_fmt(std::integral_constant<int, 64>{});
        case 128: return by_fmt(std::integral_constant<int, 128>{});
        case 256: return by_fmt(std::integral_constant<int, 256>{});
        default: return fail("paged decode attention supports head dims 64, 128 and 256");
    }
}

struct Launch {
    hipStream_t stream;
    const PagedParams* p;
    template <int D, int FMT, int NB>
    int run() const {
        const Instance in = kernel_of<D, FMT, NB>(p->page_list != nullptr);
        hipLaunchKernelGGL(in.kernel, dim3(p->grid), dim3(64 * in.waves), 0, stream, *p);
        return check_launch("paged_attention_kernel");
    }
};

struct Occupancy {
    int* per_cu;
    int* waves;
    template <int D, int FMT, int NB>
    int run() const {
        int blocks = 0;
        const Instance in = kernel_of<D, FMT, NB>(false);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, in.kernel, 64 * in.waves, 0) != hipSuccess ||
            blocks <= 0)
            blocks = 1;
        *per_cu = blocks;
        *waves = in.waves;
        return 0;
    }
};

}  // namespace

int paged_resident_groups(int head_dim, int format, int rows, int* per_cu, int* waves) {
    return dispatch(head_dim, format, rows, Occupancy{per_cu, waves});
}

int paged_attention(const PagedParams& p, hipStream_t stream) {
    return dispatch(p.head_dim, p.kv_format, p.rows, Launch{stream, &p});
}

}  // namespace eco
