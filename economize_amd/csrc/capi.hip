// extern "C" entry points of libeconomize_amd.so (declared in include/economize_amd.h): argument validation, launch
// plans and error reporting around the kernels.

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/economize_amd.h"
#include "common.hpp"
#include "dense_attention.hpp"
#include "gather.hpp"
#include "kivi.hpp"
#include "kivi_cells.hpp"
#include "kivi_dense.hpp"
#include "kv_quant.hpp"
#include "paged_attention.hpp"
#include "quest.hpp"

namespace eco {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& message) { g_error = message; }

int fail(const std::string& message) {
    set_error(message);
    return 1;
}

int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error(std::string(what) + ": " + hipGetErrorString(err));
        return 2;
    }
    return 0;
}

namespace {

int device_cus() {
    static int cached[64] = {0};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
    if (cached[device] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
            cus = 256;
        cached[device] = cus;
    }
    return cached[device];
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// The attention kernels hold at most 64 query rows per KV head (four column blocks of 16). A call with more (query
// heads per KV head x queries, at most 64 heads per KV head) is launched in query chunks of floor(64 / groups), one
// after the other on the stream, each chunk's causal limits shifted by the queries after it (query qi of Q sees the
// tokens below L - Q + qi + 1).
struct QueryChunks {
    int per, count, last;  // queries per chunk, chunks, queries of the last chunk
};

QueryChunks query_chunks(int groups, int queries) {
    QueryChunks c;
    c.per = std::min(std::max(1, 64 / std::max(groups, 1)), queries);
    c.count = (queries + c.per - 1) / c.per;
    c.last = queries - (c.count - 1) * c.per;
    return c;
}

// Workgroups of a launch: every CU's resident workgroups of the kernel instance, but at least four tiles (256 tokens)
// per wave over the longest possible tile sequence, which bounds the partials a row can be cut into
// (ECO_PAGED_GRID overrides the count for tuning).
int paged_grid(int batch, int kv_heads, int rows, int head_dim, int format, int max_seq_len, int listed, int span) {
    static const int forced = [] {
        const char* env = std::getenv("ECO_PAGED_GRID");
        return env ? std::atoi(env) : 0;
    }();
    // cache pages a row reads: every page, or with a page list the listed pages and a tail of about one list page
    // (rows whose tail is longer only get more tiles per wave)
    const int64_t dense = (max_seq_len + 15) / 16;
    const int64_t row_pages = listed > 0 ? std::min<int64_t>(dense, listed + span + 1) : dense;
    const int64_t tiles = static_cast<int64_t>(batch) * kv_heads * ((row_pages + 3) / 4);
    int per_cu = 1, waves = 1;
    if (paged_resident_groups(head_dim, format, rows, &per_cu, &waves)) return 0;
    if (forced > 0) return forced;
    const int64_t cus = device_cus();
    int64_t grid = cus * per_cu;
    const int64_t cap = (tiles + 4 * waves - 1) / (4 * waves);  // at least four tiles per wave
    grid = grid < cap ? grid : cap;
    // little work (Quest's selected pages, short rows): one workgroup per CU with at least a tile per wave, which
    // beats fewer, longer ranges even with the cross-workgroup merges (Quest at B=8, 64 pages: 48.6 us at 256
    // workgroups against 53.2 us at one workgroup per row)
    if (grid < cus) {
        const int64_t spread = (tiles + waves - 1) / waves;
        grid = spread < cus ? spread : cus;
    }
    return static_cast<int>(grid < 1 ? 1 : grid);
}

// Workspace: row counters [B * Hkv] int32 (zero before the first call; every call leaves them zero), then two
// partial slots per wave, each [rows, D + 2] floats (maxima, sums, accumulators).
struct Workspace {
    size_t counter_bytes, part_bytes;
    size_t total() const { return counter_bytes + part_bytes; }
};

Workspace paged_workspace(int batch, int kv_heads, int rows, int head_dim, int grid) {
    return Workspace{align256(static_cast<size_t>(batch) * kv_heads * sizeof(int32_t)),
                     align256(static_cast<size_t>(2) * grid * rows * (head_dim + 2) * sizeof(float))};
}

// The KIVI decode launch: as paged_grid, over 32-token tiles.
int kivi_grid(int batch, int kv_heads, int rows, int head_dim, int bits, int max_seq_len) {
    static const int forced = [] {
        const char* env = std::getenv("ECO_KIVI_GRID");
        return env ? std::atoi(env) : 0;
    }();
    const int64_t tiles = static_cast<int64_t>(batch) * kv_heads * ((max_seq_len + 31) / 32);
    int per_cu = 1, waves = 1;
    if (kivi_resident_groups(head_dim, bits, rows, &per_cu, &waves)) return 0;
    int64_t grid = forced > 0 ? forced : static_cast<int64_t>(device_cus()) * per_cu;
    const int64_t cap = (tiles + 4 * waves - 1) / (4 * waves);  // at least four tiles per wave
    grid = grid < cap ? grid : cap;
    return static_cast<int>(grid < 1 ? 1 : grid);
}

// The dense decode launch plan, a function of the shapes only: blocks of 16 query rows, and the key axis cut into
// splits (multiples of 32 keys) so that about eight waves per CU run. Workspace: a counter per block (int32, zero
// before the first call; every call leaves them zero), then each block's split partials [splits][16][D + 2] floats.
struct DensePlan {
    int m_tiles, splits, padded_dim;
    size_t counter_bytes, workspace;
};

DensePlan dense_plan(int batch, int queries, int q_heads, int kv_heads, int keys, int head_dim, int value_dim) {
    DensePlan d{};
    const int rows = (q_heads / kv_heads) * queries;
    d.m_tiles = (rows + 15) / 16;
    d.padded_dim = dense_padded_dim(head_dim, value_dim);
    const int64_t programs = static_cast<int64_t>(batch) * kv_heads * d.m_tiles;
    const int64_t tiles = (std::max(keys, 1) + 31) / 32;
    // waves per CU the splits aim at (ECO_DENSE_WAVES overrides it for tuning)
    static const int per_cu = [] {
        const char* env = std::getenv("ECO_DENSE_WAVES");
        return env && std::atoi(env) > 0 ? std::atoi(env) : 8;
    }();
    int64_t splits = (per_cu * static_cast<int64_t>(device_cus()) + programs - 1) / programs;
    splits = std::max<int64_t>(1, std::min(splits, tiles));
    // as many splits as an even share of the tiles needs (split s takes tiles s, s + splits, ...)
    const int64_t share = (tiles + splits - 1) / splits;
    d.splits = static_cast<int>((tiles + share - 1) / share);
    d.counter_bytes = align256(static_cast<size_t>(programs) * sizeof(int32_t));
    d.workspace = d.counter_bytes +
                  align256(static_cast<size_t>(programs) * d.splits * 16 * (d.padded_dim + 2) * sizeof(float));
    return d;
}

int element_bytes(int format) { return format == FP32 ? 4 : (format == BF16 || format == FP16 ? 2 : 1); }

int check_kivi_shape(int head_dim, int bits, int group) {
    if (group != 32) return fail("kivi: the paged cache takes groups of 32 (key tokens and value channels)");
    if (bits != 2 && bits != 4) return fail("kivi: codes must have 2 or 4 bits");
    if (head_dim != 64 && head_dim != 128) return fail("kivi: head dim must be 64 or 128");
    return 0;
}

int run_paged_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* k_cache,
                     const void* v_cache, int32_t kv_format, int32_t num_pages, const float* k_scale,
                     const float* v_scale, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                     const int32_t* seq_lens, const int32_t* page_list, int64_t pl_b, int64_t pl_h, int32_t n_sel,
                     int32_t list_page_size, const int32_t* done, const float* sinks, void* out, int64_t so_b,
                     int64_t so_q, int64_t so_h, int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                     int32_t head_dim, int32_t page_size, int32_t max_seq_len, float scale, float softcap,
                     const uint32_t* mask_bits, int64_t mk_b, int64_t mk_h, int64_t mk_q, int32_t mask_words,
                     void* workspace, size_t workspace_bytes, void* stream, bool validate_only = false) {
    if (!q || !k_cache || !v_cache || !block_table || !seq_lens || !out)
        return fail("paged decode: null q, cache, block table, seq_lens or out pointer");
    if (batch <= 0 || queries <= 0 || q_heads <= 0 || kv_heads <= 0 || num_pages <= 0 || bt_cols <= 0)
        return fail("paged decode: batch, queries, heads, pages and block-table columns must be positive");
    if (bt_stride < bt_cols) return fail("paged decode: block-table stride is smaller than its column count");
    if (q_heads % kv_heads) return fail("paged decode: query heads are not a multiple of the KV heads");
    if (page_size != 16) return fail("paged decode: pages must hold 16 tokens");
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail("paged decode: head dim must be 64, 128 or 256");
    if (kv_format != BF16 && kv_format != FP8_E4M3 && kv_format != FP8_E5M2)
        return fail("paged decode: KV format must be bf16, fp8 e4m3 or fp8 e5m2");
    if (q_format != BF16 && q_format != FP16) return fail("paged decode: queries must be bf16 or fp16");
    if (q_format == FP16 && (kv_format == BF16 || page_list))
        return fail("paged decode: fp16 queries read an fp8 cache, without a page list");
    const int groups = q_heads / kv_heads;
    if (groups > 64) return fail("paged decode: at most 64 query heads per KV head");
    const QueryChunks qc = query_chunks(groups, queries);
    if ((reinterpret_cast<uintptr_t>(q) & 15) || (sq_b & 7) || (sq_q & 7) || (sq_h & 7))
        return fail("paged decode: the query must be 16-byte aligned with strides that are multiples of 8");
    if (page_list && (!done || n_sel < 0)) return fail("paged decode: a page list needs done[] and n_sel >= 0");
    if (list_page_size == 0) list_page_size = 16;
    if (list_page_size < 16 || list_page_size % 16)
        return fail("paged decode: listed pages must hold a positive multiple of 16 tokens");
    const int span = list_page_size / 16;
    if (max_seq_len <= 0) return fail("paged decode: max_seq_len must be positive");
    if (!(scale == scale)) return fail("paged decode: scale is NaN");
    if (mask_bits && mask_words <= 0) return fail("paged decode: a mask needs a positive word count");

    // the launch plan of each chunk shape (every chunk but the last, then the last)
    const int listed = page_list ? n_sel * span : 0;
    int grids[2];
    size_t need = 0;
    for (int i = 0; i < 2; ++i) {
        const int rows_i = groups * (i == 0 ? qc.per : qc.last);
        grids[i] = paged_grid(batch, kv_heads, rows_i, head_dim, kv_format, max_seq_len, listed, span);
        if (grids[i] <= 0) return 1;
        need = std::max(need, paged_workspace(batch, kv_heads, rows_i, head_dim, grids[i]).total());
    }
    if (validate_only) return 0;
    if (!workspace || workspace_bytes < need)
        return fail("paged decode: workspace too small (" + std::to_string(workspace_bytes) + " < " +
                    std::to_string(need) + " bytes)");

    const int es = kv_format == BF16 ? 2 : 1;
    PagedParams p;
    std::memset(&p, 0, sizeof(p));
    p.q = static_cast<const uint16_t*>(q);
    p.out_f16 = q_format == FP16;
    p.sq_b = sq_b;
    p.sq_q = sq_q;
    p.sq_h = sq_h;
    p.k_cache = static_cast<const uint8_t*>(k_cache);
    p.v_cache = static_cast<const uint8_t*>(v_cache);
    p.kc_head = static_cast<int64_t>(head_dim) * 16 * es;
    p.kc_page = p.kc_head * kv_heads;
    p.vc_head = p.kc_head;
    p.vc_page = p.kc_page;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.num_pages = num_pages;
    p.seq_lens = seq_lens;
    p.page_list = page_list;
    p.pl_b = pl_b;
    p.pl_h = pl_h;
    p.n_sel = page_list ? n_sel : 0;
    p.span = span;
    p.done = done;
    p.k_scale = k_scale;
    p.v_scale = v_scale;
    p.sinks = sinks;
    p.mask = mask_bits;
    p.mk_b = mk_b;
    p.mk_h = mk_h;
    p.mk_q = mk_q;
    p.mask_words = mask_bits ? mask_words : 0;
    char* base = static_cast<char*>(workspace);
    p.counters = reinterpret_cast<int32_t*>(base);
    p.part = reinterpret_cast<float*>(base + paged_workspace(batch, kv_heads, 1, head_dim, 1).counter_bytes);
    p.so_b = so_b;
    p.so_q = so_q;
    p.so_h = so_h;
    p.batch = batch;
    p.q_heads = q_heads;
    p.kv_heads = kv_heads;
    p.groups = groups;
    p.head_dim = head_dim;
    p.kv_format = kv_format;
    p.scale = scale;
    p.softcap = softcap > 0.0f ? softcap : 0.0f;
    for (int c = 0; c < qc.count; ++c) {
        const int q0 = c * qc.per, k = c + 1 < qc.count ? qc.per : qc.last;
        p.q = static_cast<const uint16_t*>(q) + q0 * sq_q;
        p.out = static_cast<uint16_t*>(out) + q0 * so_q;
        p.mask = mask_bits ? mask_bits + q0 * mk_q : nullptr;
        p.queries = k;
        p.queries_after = queries - q0 - k;
        p.rows = groups * k;
        p.grid = grids[c + 1 < qc.count ? 0 : 1];
        const int rc = p.out_f16 ? paged_attention_f16(p, static_cast<hipStream_t>(stream))
                                 : paged_attention(p, static_cast<hipStream_t>(stream));
        if (rc) return rc;
    }
    return 0;
}

// ---- the static scratch of eco_paged_decode_static ---------------------------------------------------------------
// A workspace that needs no allocation: one array per GPU, held until the process ends. Its host-side name is a
// stand-in, not a device address: host code uses only the address hipGetSymbolAddress returns for the current
// device (scratch_on_device), never the array's name.
constexpr size_t kScratchBytes = size_t(32) << 20;  // 32 MiB
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// bits[((b * heads + h) * queries + q) * words + w] bit k = mask[b, h, q, 32 w + k] != 0 (0 past the keys).
__global__ void mask_bits_kernel(const uint8_t* mask, int64_t sm_b, int64_t sm_h, int64_t sm_q, int64_t sm_s,
                                 int batch, int heads, int queries, int keys, uint32_t* bits, int words) {
    const int64_t total = static_cast<int64_t>(batch) * heads * queries * words;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int w = static_cast<int>(i % words);
        const int64_t row = i / words;
        const int q = static_cast<int>(row % queries);
        const int h = static_cast<int>((row / queries) % heads);
        const int b = static_cast<int>(row / (static_cast<int64_t>(queries) * heads));
        const uint8_t* src = mask + b * sm_b + h * sm_h + q * sm_q;
        uint32_t word = 0;
        for (int k = 0; k < 32; ++k) {
            const int t = 32 * w + k;
            if (t < keys && src[static_cast<int64_t>(t) * sm_s]) word |= 1u << k;
        }
        bits[i] = word;
    }
}

__global__ void zero_words_kernel(uint32_t* words, int count) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) words[i] = 0;
}

// The device address of scratch on the current device (looked up once per device), or null with the error set.
void* scratch_on_device() {
    static std::mutex lock;
    static void* addresses[64] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
        set_error("paged decode (static scratch): no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> guard(lock);
    if (!addresses[device]) {
        void* ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !ptr) {
            set_error(std::string("paged decode (static scratch): hipGetSymbolAddress failed: ") +
                      hipGetErrorString(err));
            return nullptr;
        }
        addresses[device] = ptr;
    }
    return addresses[device];
}

// The compact entries of a gathered cache (the reference's GatheredKV, attention/gathered.py:39-64).
struct GatheredArgs {
    const void* ck;
    const void* cv;
    int64_t sck_b, sck_h, sck_s, scv_b, scv_h, scv_s;
    const int32_t* index;
    int64_t si_b, si_h;
    const int32_t* count;
    const int32_t* start;
    int capacity, dropped;
};

// The selected pages of a Quest call over a dense cache (the reference's quest_decode_attention arguments,
// attention/quest.py:239-344): index [B, Hkv, pages], done [B], pages of 2^shift slots, min(done) for the plan.
struct QuestListArgs {
    const int32_t* index;
    int64_t si_b, si_h;
    int pages, shift, min_done;
    const int32_t* done;
};

// The codes of a KIVI packed call (the reference's KIVIPacked record, attention/kivi.py:80-132).
struct KiviPackedArgs {
    const uint8_t* kc;
    int64_t skc_b, skc_h, skc_s;
    const uint16_t* ks;
    const uint16_t* kz;
    int64_t sks_b, sks_h, sks_g;
    const uint8_t* vc;
    int64_t svc_b, svc_h, svc_s;
    const uint16_t* vs;
    const uint16_t* vz;
    int64_t svs_b, svs_h, svs_s;
    const int32_t* kq;
    const int32_t* vq;
    int bits, key_group, value_group, ring;
};

int dense_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
               const void* v, int32_t kv_format, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b, int64_t sv_h,
               int64_t sv_s, const float* k_scale, const float* v_scale, const uint8_t* mask, int64_t sm_b,
               int64_t sm_h, int64_t sm_q, int64_t sm_s, const float* sinks, void* out, int64_t so_b, int64_t so_q,
               int64_t so_h, int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys,
               int32_t head_dim, int32_t value_dim, float scale, float softcap, void* workspace,
               size_t workspace_bytes, void* stream, const GatheredArgs* g, const QuestListArgs* ql = nullptr,
               const KiviPackedArgs* kp = nullptr) {
    if (!q || !k || !v || !out) return fail("decode: null query, key, value or output pointer");
    if (batch <= 0 || queries <= 0 || q_heads <= 0 || kv_heads <= 0 || keys < 0)
        return fail("decode: batch, queries and heads must be positive, keys non-negative");
    if (q_heads % kv_heads)
        return fail("decode: " + std::to_string(q_heads) + " query heads are not a multiple of " +
                    std::to_string(kv_heads) + " KV heads");
    if (q_format != BF16 && q_format != FP16 && q_format != FP32)
        return fail("decode: queries must be bf16, fp16 or fp32");
    const bool fp8 = kv_format == FP8_E4M3 || kv_format == FP8_E5M2;
    if (kv_format != q_format && !fp8) return fail("decode: K/V must be in the query's dtype or fp8");
    if ((k_scale || v_scale) && !fp8) return fail("decode: per-head scales apply to fp8 K/V only");
    const int es = element_bytes(kv_format), qs = element_bytes(q_format);
    for (int dim : {head_dim, value_dim})
        if (dim <= 0 || dim % 8 || (dim * es) % 16 || dim > (es == 4 ? 256 : 512))
            return fail("decode: head dims must be positive multiples of 8 (of 16 for fp8), at most 512 (256 for fp32)");
    auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!aligned(q) || !aligned(k) || !aligned(v))
        return fail("decode: query, key and value must be 16-byte aligned");
    for (int64_t st : {sq_b, sq_h, sq_q})
        if ((st * qs) % 16) return fail("decode: query strides must be multiples of 16 bytes");
    for (int64_t st : {sk_b, sk_h, sk_s, sv_b, sv_h, sv_s})
        if ((st * es) % 16) return fail("decode: key and value strides must be multiples of 16 bytes");
    if (!(scale == scale)) return fail("decode: scale is NaN");
    // the virtual key axis: gathered, keys - dropped; Quest, the selected pages' slots and the longest tail
    int plan_keys = g ? std::max(1, keys - g->dropped) : keys;
    if (ql)
        plan_keys = static_cast<int>(std::max<int64_t>(
            1, (static_cast<int64_t>(ql->pages) << ql->shift) + keys - (static_cast<int64_t>(ql->min_done) << ql->shift)));
    const DensePlan d = dense_plan(batch, queries, q_heads, kv_heads, plan_keys, head_dim, value_dim);
    if (!workspace || workspace_bytes < d.workspace)
        return fail("decode: workspace too small (" + std::to_string(workspace_bytes) + " < " +
                    std::to_string(d.workspace) + " bytes)");
    DenseParams p;
    std::memset(&p, 0, sizeof(p));
    p.q = q;
    p.sq_b = sq_b;
    p.sq_h = sq_h;
    p.sq_q = sq_q;
    p.q_format = q_format;
    p.k = k;
    p.v = v;
    p.kv_format = kv_format;
    p.sk_b = sk_b;
    p.sk_h = sk_h;
    p.sk_s = sk_s;
    p.sv_b = sv_b;
    p.sv_h = sv_h;
    p.sv_s = sv_s;
    p.k_scale = k_scale;
    p.v_scale = v_scale;
    p.mask = mask;
    p.sm_b = sm_b;
    p.sm_h = sm_h;
    p.sm_q = sm_q;
    p.sm_s = sm_s;
    p.sinks = sinks;
    p.out = out;
    p.so_b = so_b;
    p.so_q = so_q;
    p.so_h = so_h;
    p.counters = static_cast<int32_t*>(workspace);
    p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + d.counter_bytes);
    p.batch = batch;
    p.queries = queries;
    p.q_heads = q_heads;
    p.kv_heads = kv_heads;
    p.groups = q_heads / kv_heads;
    p.rows = p.groups * queries;
    p.keys = plan_keys;
    p.dense_keys = keys;
    p.head_dim = head_dim;
    p.value_dim = value_dim;
    p.m_tiles = d.m_tiles;
    p.splits = d.splits;
    p.scale = scale;
    p.softcap = softcap > 0.0f ? softcap : 0.0f;
    if (g) {
        p.gk = g->ck;
        p.gv = g->cv;
        p.sgk_b = g->sck_b;
        p.sgk_h = g->sck_h;
        p.sgk_s = g->sck_s;
        p.sgv_b = g->scv_b;
        p.sgv_h = g->scv_h;
        p.sgv_s = g->scv_s;
        p.g_index = g->index;
        p.sgi_b = g->si_b;
        p.sgi_h = g->si_h;
        p.g_count = g->count;
        p.g_start = g->start;
        p.g_capacity = g->capacity;
    }
    if (ql) {
        p.qp_list = ql->index;
        p.sqp_b = ql->si_b;
        p.sqp_h = ql->si_h;
        p.qp_pages = ql->pages;
        p.qp_shift = ql->shift;
        p.qp_done = ql->done;
    }
    if (kp) {
        p.kp_kc = kp->kc;
        p.skc_b = kp->skc_b;
        p.skc_h = kp->skc_h;
        p.skc_s = kp->skc_s;
        p.kp_ks = kp->ks;
        p.kp_kz = kp->kz;
        p.sks_b = kp->sks_b;
        p.sks_h = kp->sks_h;
        p.sks_g = kp->sks_g;
        p.kp_vc = kp->vc;
        p.svc_b = kp->svc_b;
        p.svc_h = kp->svc_h;
        p.svc_s = kp->svc_s;
        p.kp_vs = kp->vs;
        p.kp_vz = kp->vz;
        p.svs_b = kp->svs_b;
        p.svs_h = kp->svs_h;
        p.svs_s = kp->svs_s;
        p.kp_kq = kp->kq;
        p.kp_vq = kp->vq;
        p.kp_bits = kp->bits;
        p.kp_kg = kp->key_group;
        p.kp_vg = kp->value_group;
        p.kp_ring = kp->ring;
        return kivi_packed_attention(p, d.padded_dim, static_cast<hipStream_t>(stream));
    }
    return dense_attention(p, d.padded_dim, static_cast<hipStream_t>(stream));
}


// The cell layout of layout.py:196-213 and CellLayout's offsets (layout.py:133-193); 1 (with a message) when the
// head size or the bits do not fit KIVI's packing.
int make_cell_layout(int head_dim, int element_size, int bits, int group, CellLayout* out) {
    if (bits != 2 && bits != 4 && bits != 8) return fail("kivi cells: bits must be 2, 4 or 8");
    if (head_dim < 16 || head_dim > 256 || (head_dim & (head_dim - 1)))
        return fail("kivi cells: the head size must be a power of two from 16 to 256");
    if (group < 1 || group > 128 || (group & (group - 1)))
        return fail("kivi cells: the group size must be a power of two of at most 128");
    if (element_size != 2 && element_size != 4) return fail("kivi cells: the cache dtype must be bf16, fp16 or fp32");
    CellLayout L;
    L.head_dim = head_dim;
    L.element_size = element_size;
    L.bits = bits;
    L.group = group;
    L.value_group = head_dim % group == 0 ? group : head_dim;
    L.key_aux = (2 * head_dim + group - 1) / group;
    const int nvg = head_dim / L.value_group, code_bytes = head_dim / (8 / bits);
    L.off_v = head_dim * element_size;
    L.off_vs = 2 * head_dim * element_size;
    L.off_vz = L.off_vs + 2 * nvg;
    L.off_ka = L.off_vz + 2 * nvg;
    L.off_kc = L.off_ka + 2 * L.key_aux;
    L.off_vc = L.off_kc + code_bytes;
    L.off_flag = L.off_vc + code_bytes;
    L.size = (L.off_flag + 2 + 15) / 16 * 16;
    *out = L;
    return 0;
}

}  // namespace

}  // namespace eco

using namespace eco;

// The append's arguments as AppendParams (1 with a message when they are invalid; tokens may be 0).
static int append_params(const void* k_new, const void* v_new, int32_t in_format, int64_t sk_t, int64_t sk_h,
                         int64_t sv_t, int64_t sv_h, const int32_t* slot_mapping, int32_t tokens, void* k_cache,
                         void* v_cache, int32_t num_pages, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                         int32_t cache_format, const float* k_scale, const float* v_scale, AppendParams& p) {
    if (tokens < 0) return fail("paged append: negative token count");
    if ((tokens > 0 && (!k_new || !v_new || !slot_mapping)) || !k_cache || !v_cache)
        return fail("paged append: null input, slot mapping or cache pointer");
    if (in_format != BF16 && in_format != FP16 && in_format != FP32)
        return fail("paged append: inputs must be bf16, fp16 or fp32");
    if (cache_format != BF16 && cache_format != FP8_E4M3 && cache_format != FP8_E5M2)
        return fail("paged append: cache format must be bf16, fp8 e4m3 or fp8 e5m2");
    if (page_size != 16) return fail("paged append: pages must hold 16 tokens");
    if (head_dim <= 0 || head_dim % 16 || kv_heads <= 0 || num_pages <= 0)
        return fail("paged append: head dim must be a positive multiple of 16, heads and pages positive");
    if (cache_format == BF16 && (k_scale || v_scale)) return fail("paged append: a bf16 cache takes no scales");
    const int es = cache_format == BF16 ? 2 : 1;
    p.k_new = k_new;
    p.v_new = v_new;
    p.in_format = in_format;
    p.sk_t = sk_t;
    p.sk_h = sk_h;
    p.sv_t = sv_t;
    p.sv_h = sv_h;
    p.slots = slot_mapping;
    p.tokens = tokens;
    p.k_cache = static_cast<uint8_t*>(k_cache);
    p.v_cache = static_cast<uint8_t*>(v_cache);
    p.kc_head = static_cast<int64_t>(head_dim) * 16 * es;
    p.kc_page = p.kc_head * kv_heads;
    p.vc_head = p.kc_head;
    p.vc_page = p.kc_page;
    p.kv_heads = kv_heads;
    p.head_dim = head_dim;
    p.num_pages = num_pages;
    p.cache_format = cache_format;
    p.k_scale = k_scale;
    p.v_scale = v_scale;
    return 0;
}

extern "C" {

const char* eco_last_error(void) { return g_error.c_str(); }

int eco_abi_version(void) { return 8; }

int eco_paged_append(const void* k_new, const void* v_new, int32_t in_format, int64_t sk_t, int64_t sk_h,
                     int64_t sv_t, int64_t sv_h, const int32_t* slot_mapping, int32_t tokens, void* k_cache,
                     void* v_cache, int32_t num_pages, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                     int32_t cache_format, const float* k_scale, const float* v_scale, void* stream) {
    if (tokens == 0) return 0;
    AppendParams p;
    if (int rc = append_params(k_new, v_new, in_format, sk_t, sk_h, sv_t, sv_h, slot_mapping, tokens, k_cache, v_cache,
                               num_pages, kv_heads, head_dim, page_size, cache_format, k_scale, v_scale, p))
        return rc;
    return paged_append(p, static_cast<hipStream_t>(stream));
}

int eco_paged_append_quest(const void* k_new, const void* v_new, int32_t in_format, int64_t sk_t, int64_t sk_h,
                           int64_t sv_t, int64_t sv_h, const int32_t* slot_mapping, int32_t tokens, void* k_cache,
                           void* v_cache, int32_t num_pages, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                           int32_t cache_format, const float* k_scale, const float* v_scale,
                           const int32_t* block_table, int64_t bt_stride, int32_t bt_cols, const int32_t* committed,
                           int32_t* valid, int32_t* done, int32_t* counters, int32_t quest_page_size, void* kmin,
                           void* kmax, int64_t sb_b, int64_t sb_h, int64_t sb_p, int32_t page_cap, int32_t batch,
                           void* stream) {
    AppendParams p;
    if (int rc = append_params(k_new, v_new, in_format, sk_t, sk_h, sv_t, sv_h, slot_mapping, tokens, k_cache, v_cache,
                               num_pages, kv_heads, head_dim, page_size, cache_format, k_scale, v_scale, p))
        return rc;
    if (!block_table || !committed || !valid || !counters || !kmin || !kmax)
        return fail("paged append (quest): null block table, committed, valid, counters or bounds");
    if (batch <= 0 || bt_cols <= 0 || bt_stride < bt_cols || page_cap < 0)
        return fail("paged append (quest): batch and block-table columns must be positive");
    if (quest_page_size < 16 || quest_page_size % 16 || (quest_page_size & (quest_page_size - 1)))
        return fail("paged append (quest): quest pages must hold a power of two of at least 16 tokens");
    const int es = cache_format == BF16 ? 2 : 1;
    if ((head_dim * es) % 64) return fail("paged append (quest): head dim must fill whole runs");
    BoundsParams q;
    q.k_cache = p.k_cache;
    q.kc_head = p.kc_head;
    q.kc_page = p.kc_page;
    q.kv_format = cache_format;
    q.num_pages = num_pages;
    q.block_table = block_table;
    q.bt_stride = bt_stride;
    q.bt_cols = bt_cols;
    q.first = 0;
    q.last = 0;
    q.span = quest_page_size / 16;
    q.kmin = static_cast<uint16_t*>(kmin);
    q.kmax = static_cast<uint16_t*>(kmax);
    q.sb_b = sb_b;
    q.sb_h = sb_h;
    q.sb_p = sb_p;
    q.batch = batch;
    q.kv_heads = kv_heads;
    q.head_dim = head_dim;
    q.committed = committed;
    q.valid = valid;
    q.done = done;
    q.page_cap = page_cap;
    return paged_append_quest(p, q, counters, static_cast<hipStream_t>(stream));
}

int eco_fp8_encode(const void* src, int32_t in_format, int64_t ss_b, int64_t ss_h, int64_t ss_t, void* dst,
                   int32_t out_format, int64_t sd_b, int64_t sd_h, int64_t sd_t, int32_t batch, int32_t heads,
                   int32_t tokens, int32_t head_dim, const float* head_scale, float* token_scale, int64_t st_b,
                   int64_t st_h, int64_t st_t, void* stream) {
    if (batch < 0 || heads < 0 || tokens < 0) return fail("fp8 encode: negative shape");
    if (head_dim <= 0 || head_dim > 512) return fail("fp8 encode: head dim must be in 1..512");
    if (static_cast<int64_t>(batch) * heads * tokens == 0) return 0;
    if (!src || !dst) return fail("fp8 encode: null source or destination");
    if (in_format != BF16 && in_format != FP16 && in_format != FP32)
        return fail("fp8 encode: the source must be bf16, fp16 or fp32");
    if (out_format != FP8_E4M3 && out_format != FP8_E5M2)
        return fail("fp8 encode: the output format must be fp8 e4m3 or e5m2");
    if (head_scale && token_scale) return fail("fp8 encode: per-head and per-token scales exclude each other");
    EncodeParams p{src, in_format, ss_b, ss_h, ss_t, static_cast<uint8_t*>(dst), out_format, sd_b, sd_h, sd_t,
                   batch, heads, tokens, head_dim, head_scale, token_scale, st_b, st_h, st_t};
    return fp8_encode(p, static_cast<hipStream_t>(stream));
}

int eco_kv_head_absmax(const void* x, int32_t in_format, int32_t a, int32_t h, int32_t s, int32_t d, int64_t sa,
                       int64_t sh, int64_t ss, int64_t sd, uint32_t* absmax_bits, void* stream) {
    if (!x || !absmax_bits) return fail("head absmax: null pointer");
    if (in_format != BF16 && in_format != FP16 && in_format != FP32)
        return fail("head absmax: input must be bf16, fp16 or fp32");
    if (a < 0 || h <= 0 || s < 0 || d <= 0) return fail("head absmax: bad shape");
    if (a == 0 || s == 0) return 0;
    AbsmaxParams p{x, in_format, a, h, s, d, sa, sh, ss, sd, absmax_bits};
    return head_absmax(p, static_cast<hipStream_t>(stream));
}

int eco_fp8_scales_from_absmax(const uint32_t* absmax_bits, int32_t heads, int32_t format, float* scales,
                               void* stream) {
    if (!absmax_bits || !scales || heads <= 0) return fail("fp8 scales: null pointer or no heads");
    if (format != FP8_E4M3 && format != FP8_E5M2) return fail("fp8 scales: format must be fp8 e4m3 or e5m2");
    return scales_from_absmax(absmax_bits, heads, format, scales, static_cast<hipStream_t>(stream));
}

size_t eco_paged_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                                       int32_t head_dim, int32_t max_seq_len, int32_t n_sel, int32_t list_page_size,
                                       int32_t kv_format) {
    if (batch <= 0 || queries <= 0 || kv_heads <= 0 || q_heads <= 0 || head_dim <= 0 || max_seq_len <= 0) return 0;
    const int groups = q_heads / kv_heads;
    const QueryChunks qc = query_chunks(groups, queries);
    const int span = list_page_size >= 16 ? list_page_size / 16 : 1;
    size_t need = 0;
    for (const int k : {qc.per, qc.last}) {
        const int grid =
            paged_grid(batch, kv_heads, groups * k, head_dim, kv_format, max_seq_len, n_sel > 0 ? n_sel * span : 0, span);
        if (grid <= 0) return 0;
        need = std::max(need, paged_workspace(batch, kv_heads, groups * k, head_dim, grid).total());
    }
    return need;
}

int eco_paged_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* k_cache,
                     const void* v_cache, int32_t kv_format, int32_t num_pages, const float* k_scale,
                     const float* v_scale, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                     const int32_t* seq_lens, const int32_t* page_list, int64_t pl_b, int64_t pl_h, int32_t n_sel,
                     int32_t list_page_size, const int32_t* done, const float* sinks, void* out, int64_t so_b,
                     int64_t so_q, int64_t so_h, int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                     int32_t head_dim, int32_t page_size, int32_t max_seq_len, float scale, float softcap,
                     const uint32_t* mask_bits, int64_t mk_b, int64_t mk_h, int64_t mk_q, int32_t mask_words,
                     void* workspace, size_t workspace_bytes, void* stream) {
    return run_paged_decode(q, q_format, sq_b, sq_q, sq_h, k_cache, v_cache, kv_format, num_pages, k_scale, v_scale,
                            block_table, bt_stride, bt_cols, seq_lens, page_list, pl_b, pl_h, n_sel, list_page_size,
                            done, sinks, out, so_b, so_q, so_h, batch, queries, q_heads, kv_heads, head_dim, page_size,
                            max_seq_len, scale, softcap, mask_bits, mk_b, mk_h, mk_q, mask_words, workspace,
                            workspace_bytes, stream);
}

int eco_paged_decode_static(const void* q, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* k_cache,
                            const void* v_cache, int32_t kv_format, int32_t num_pages, const float* k_scale,
                            const float* v_scale, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                            const int32_t* seq_lens, const int32_t* page_list, int64_t pl_b, int64_t pl_h,
                            int32_t n_sel, int32_t list_page_size, const int32_t* done, const float* sinks, void* out,
                            int64_t so_b, int64_t so_q, int64_t so_h, int32_t batch, int32_t queries,
                            int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                            int32_t max_seq_len, float scale, float softcap, const uint32_t* mask_bits, int64_t mk_b,
                            int64_t mk_h, int64_t mk_q, int32_t mask_words, void* stream) {
    // every argument is checked before anything is launched
    if (const int rc = run_paged_decode(q, BF16, sq_b, sq_q, sq_h, k_cache, v_cache, kv_format, num_pages, k_scale,
                                        v_scale,
                                        block_table, bt_stride, bt_cols, seq_lens, page_list, pl_b, pl_h, n_sel,
                                        list_page_size, done, sinks, out, so_b, so_q, so_h, batch, queries, q_heads,
                                        kv_heads, head_dim, page_size, max_seq_len, scale, softcap, mask_bits, mk_b,
                                        mk_h, mk_q, mask_words, nullptr, 0, stream, true))
        return rc;
    const size_t need = eco_paged_decode_workspace_size(batch, queries, q_heads, kv_heads, head_dim, max_seq_len,
                                                        page_list ? n_sel : 0, list_page_size, kv_format);
    if (need > kScratchBytes)
        return fail("paged decode (static scratch): the call needs " + std::to_string(need) +
                    " bytes of scratch, more than the library's " + std::to_string(kScratchBytes) +
                    "; use eco_paged_decode with a workspace");
    void* ptr = scratch_on_device();
    if (!ptr) return 2;
    // the row counters must be zero when the call starts (the array keeps the last call's contents): cleared by a
    // fill kernel on the call's stream (no memset node in a captured graph)
    const int words = static_cast<int>(align256(static_cast<size_t>(batch) * kv_heads * sizeof(int32_t)) / 4);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, s, static_cast<uint32_t*>(ptr),
                       words);
    if (const int rc = check_launch("zero_words_kernel")) return rc;
    return run_paged_decode(q, BF16, sq_b, sq_q, sq_h, k_cache, v_cache, kv_format, num_pages, k_scale, v_scale,
                            block_table, bt_stride, bt_cols, seq_lens, page_list, pl_b, pl_h, n_sel, list_page_size,
                            done, sinks, out, so_b, so_q, so_h, batch, queries, q_heads, kv_heads, head_dim, page_size,
                            max_seq_len, scale, softcap, mask_bits, mk_b, mk_h, mk_q, mask_words, ptr, kScratchBytes,
                            stream);
}

size_t eco_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys,
                                 int32_t head_dim, int32_t value_dim) {
    if (batch <= 0 || queries <= 0 || q_heads <= 0 || kv_heads <= 0 || keys < 0 || q_heads % kv_heads) return 0;
    if (dense_padded_dim(head_dim, value_dim) == 0) return 0;
    return dense_plan(batch, queries, q_heads, kv_heads, keys, head_dim, value_dim).workspace;
}

int eco_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
               const void* v, int32_t kv_format, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b, int64_t sv_h,
               int64_t sv_s, const float* k_scale, const float* v_scale, const uint8_t* mask, int64_t sm_b,
               int64_t sm_h, int64_t sm_q, int64_t sm_s, const float* sinks, void* out, int64_t so_b, int64_t so_q,
               int64_t so_h, int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys,
               int32_t head_dim, int32_t value_dim, float scale, float softcap, void* workspace,
               size_t workspace_bytes, void* stream) {
    return dense_decode(q, q_format, sq_b, sq_h, sq_q, k, v, kv_format, sk_b, sk_h, sk_s, sv_b, sv_h, sv_s, k_scale,
                        v_scale, mask, sm_b, sm_h, sm_q, sm_s, sinks, out, so_b, so_q, so_h, batch, queries, q_heads,
                        kv_heads, keys, head_dim, value_dim, scale, softcap, workspace, workspace_bytes, stream,
                        nullptr);
}

int eco_gathered_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
                        const void* v, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b, int64_t sv_h,
                        int64_t sv_s, const void* ck, const void* cv, int64_t sck_b, int64_t sck_h, int64_t sck_s,
                        int64_t scv_b, int64_t scv_h, int64_t scv_s, const int32_t* index, int64_t si_b,
                        int64_t si_h, const int32_t* count, const int32_t* start, int32_t capacity, int32_t dropped,
                        const uint8_t* mask, int64_t sm_b, int64_t sm_h, int64_t sm_q, int64_t sm_s,
                        const float* sinks, void* out, int64_t so_b, int64_t so_q, int64_t so_h, int32_t batch,
                        int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys, int32_t head_dim,
                        int32_t value_dim, float scale, float softcap, void* workspace, size_t workspace_bytes,
                        void* stream) {
    if (!ck || !cv || !index || !count || !start) return fail("gathered decode: null compact entries or counts");
    if (keys <= 0 || capacity < 0 || dropped < 0 || dropped > keys)
        return fail("gathered decode: need keys > 0, capacity >= 0 and 0 <= dropped <= keys");
    const int es = element_bytes(q_format);
    auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!aligned(ck) || !aligned(cv)) return fail("gathered decode: compact keys and values must be 16-byte aligned");
    for (int64_t st : {sck_b, sck_h, sck_s, scv_b, scv_h, scv_s})
        if ((st * es) % 16) return fail("gathered decode: compact strides must be multiples of 16 bytes");
    const GatheredArgs g{ck, cv, sck_b, sck_h, sck_s, scv_b, scv_h, scv_s, index, si_b, si_h, count, start,
                         capacity, dropped};
    return dense_decode(q, q_format, sq_b, sq_h, sq_q, k, v, q_format, sk_b, sk_h, sk_s, sv_b, sv_h, sv_s, nullptr,
                        nullptr, mask, sm_b, sm_h, sm_q, sm_s, sinks, out, so_b, so_q, so_h, batch, queries, q_heads,
                        kv_heads, keys, head_dim, value_dim, scale, softcap, workspace, workspace_bytes, stream, &g);
}

int eco_mask_bits(const uint8_t* mask, int64_t sm_b, int64_t sm_h, int64_t sm_q, int64_t sm_s, int32_t batch,
                  int32_t heads, int32_t queries, int32_t keys, uint32_t* bits, int32_t words, void* stream) {
    if (!mask || !bits) return fail("mask bits: null mask or output");
    if (batch <= 0 || heads <= 0 || queries <= 0 || keys < 0 || words < (keys + 31) / 32 || words <= 0)
        return fail("mask bits: sizes must be positive and words must cover the keys");
    const int64_t total = static_cast<int64_t>(batch) * heads * queries * words;
    const int blocks = static_cast<int>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(mask_bits_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), mask, sm_b,
                       sm_h, sm_q, sm_s, batch, heads, queries, keys, bits, words);
    return check_launch("mask_bits_kernel");
}

int eco_paged_gather(const void* k_cache, const void* v_cache, int32_t kv_format, int32_t num_pages,
                     const float* k_scale, const float* v_scale, const int32_t* block_table, int64_t bt_stride,
                     int32_t bt_cols, void* k_out, void* v_out, int32_t out_format, int64_t so_kb, int64_t so_kh,
                     int64_t so_ks, int64_t so_vb, int64_t so_vh, int64_t so_vs, int32_t batch, int32_t kv_heads,
                     int32_t keys, int32_t head_dim, int32_t page_size, void* stream) {
    if (!k_cache || !v_cache || !block_table || !k_out || !v_out) return fail("paged gather: null pointer");
    if (batch <= 0 || kv_heads <= 0 || keys < 0 || num_pages <= 0 || bt_cols <= 0 || bt_stride < bt_cols)
        return fail("paged gather: sizes must be positive");
    if (page_size != 16) return fail("paged gather: pages must hold 16 tokens");
    if (kv_format != BF16 && kv_format != FP8_E4M3 && kv_format != FP8_E5M2)
        return fail("paged gather: the cache must be bf16, fp8 e4m3 or fp8 e5m2");
    if (out_format != BF16 && out_format != FP16 && out_format != FP32)
        return fail("paged gather: the output must be bf16, fp16 or fp32");
    if (head_dim <= 0 || head_dim % 16) return fail("paged gather: head dim must be a positive multiple of 16");
    const int es = kv_format == BF16 ? 2 : 1;
    PagedGatherParams p{};
    p.k_cache = static_cast<const uint8_t*>(k_cache);
    p.v_cache = static_cast<const uint8_t*>(v_cache);
    p.kc_head = static_cast<int64_t>(head_dim) * 16 * es;
    p.kc_page = p.kc_head * kv_heads;
    p.vc_head = p.kc_head;
    p.vc_page = p.kc_page;
    p.kv_format = kv_format;
    p.k_scale = k_scale;
    p.v_scale = v_scale;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.num_pages = num_pages;
    p.k_out = k_out;
    p.v_out = v_out;
    p.so_kb = so_kb;
    p.so_kh = so_kh;
    p.so_ks = so_ks;
    p.so_vb = so_vb;
    p.so_vh = so_vh;
    p.so_vs = so_vs;
    p.out_format = out_format;
    p.batch = batch;
    p.kv_heads = kv_heads;
    p.keys = keys;
    p.head_dim = head_dim;
    return paged_gather(p, static_cast<hipStream_t>(stream));
}

int eco_kivi_gather(const void* blocks, int32_t num_pages, const void* k_ring, const void* v_ring, int32_t ring,
                    const int32_t* keys_quantized, const int32_t* values_quantized, const int32_t* block_table,
                    int64_t bt_stride, int32_t bt_cols, void* k_out, void* v_out, int32_t out_format, int64_t so_kb,
                    int64_t so_kh, int64_t so_ks, int64_t so_vb, int64_t so_vh, int64_t so_vs, int32_t batch,
                    int32_t kv_heads, int32_t keys, int32_t head_dim, int32_t bits, int32_t group, void* stream) {
    if (!blocks || !k_ring || !v_ring || !keys_quantized || !values_quantized || !block_table || !k_out || !v_out)
        return fail("kivi gather: null pointer");
    if (batch <= 0 || kv_heads <= 0 || keys < 0 || num_pages <= 0 || bt_cols <= 0 || bt_stride < bt_cols)
        return fail("kivi gather: sizes must be positive");
    if (int rc = check_kivi_shape(head_dim, bits, group)) return rc;
    if (ring <= 0 || ring % 32) return fail("kivi gather: the ring must hold a positive multiple of 32 slots");
    if (out_format != BF16 && out_format != FP16 && out_format != FP32)
        return fail("kivi gather: the output must be bf16, fp16 or fp32");
    const KiviLayout L{head_dim, bits};
    KiviGatherParams p{};
    p.blocks = static_cast<const uint8_t*>(blocks);
    p.blk_head = L.size();
    p.blk_page = static_cast<int64_t>(L.size()) * kv_heads;
    p.k_ring = static_cast<const uint16_t*>(k_ring);
    p.v_ring = static_cast<const uint16_t*>(v_ring);
    p.ring = ring;
    p.keys_quantized = keys_quantized;
    p.values_quantized = values_quantized;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.num_pages = num_pages;
    p.k_out = k_out;
    p.v_out = v_out;
    p.so_kb = so_kb;
    p.so_kh = so_kh;
    p.so_ks = so_ks;
    p.so_vb = so_vb;
    p.so_vh = so_vh;
    p.so_vs = so_vs;
    p.out_format = out_format;
    p.batch = batch;
    p.kv_heads = kv_heads;
    p.keys = keys;
    p.head_dim = head_dim;
    p.bits = bits;
    return kivi_gather(p, static_cast<hipStream_t>(stream));
}

size_t eco_kivi_block_bytes(int32_t head_dim, int32_t bits, int32_t group) {
    if (check_kivi_shape(head_dim, bits, group)) return 0;
    return static_cast<size_t>(KiviLayout{head_dim, bits}.size());
}

int eco_kivi_schedule(const int32_t* committed, int32_t residual, int32_t group, int32_t* keys_quantized,
                      int32_t* values_quantized, int32_t* ranges, int32_t batch, void* stream) {
    if (!committed || !keys_quantized || !values_quantized || !ranges) return fail("kivi schedule: null pointer");
    if (batch <= 0) return fail("kivi schedule: batch must be positive");
    if (group != 32 || residual <= 0 || residual % 32)
        return fail("kivi schedule: the residual length must be a positive multiple of the group (32)");
    return kivi_schedule(committed, residual, keys_quantized, values_quantized, ranges, batch,
                         static_cast<hipStream_t>(stream));
}

int eco_kivi_quantize(int32_t kind, const void* src, int32_t src_format, int64_t ss_b, int64_t ss_h, int64_t ss_t,
                      int64_t ss_d, int32_t src_start, int32_t src_ring, const int32_t* from, const int32_t* to,
                      void* blocks, int32_t num_pages, const int32_t* block_table, int64_t bt_stride,
                      int32_t bt_cols, int32_t batch, int32_t kv_heads, int32_t head_dim, int32_t bits,
                      int32_t group, int32_t max_tokens, uint32_t* overflow, void* stream) {
    if (kind != 0 && kind != 1) return fail("kivi quantize: kind must be 0 (keys) or 1 (values)");
    if (!src || !from || !to || !blocks || !block_table) return fail("kivi quantize: null pointer");
    if (src_format != BF16 && src_format != FP16 && src_format != FP32)
        return fail("kivi quantize: the source must be bf16, fp16 or fp32");
    if (batch <= 0 || kv_heads <= 0 || num_pages <= 0 || bt_cols <= 0 || bt_stride < bt_cols)
        return fail("kivi quantize: batch, heads, pages and block-table columns must be positive");
    if (int rc = check_kivi_shape(head_dim, bits, group)) return rc;
    if (src_ring < 0) return fail("kivi quantize: negative ring");
    if (max_tokens <= 0) return 0;
    const KiviLayout L{head_dim, bits};
    KiviQuantParams p;
    p.src = src;
    p.src_format = src_format;
    p.ss_b = ss_b;
    p.ss_h = ss_h;
    p.ss_t = ss_t;
    p.ss_d = ss_d;
    p.src_start = src_start;
    p.src_ring = src_ring;
    p.from = from;
    p.to = to;
    p.blocks = static_cast<uint8_t*>(blocks);
    p.blk_head = L.size();
    p.blk_page = static_cast<int64_t>(L.size()) * kv_heads;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.num_pages = num_pages;
    p.batch = batch;
    p.kv_heads = kv_heads;
    p.head_dim = head_dim;
    p.bits = bits;
    p.overflow = overflow;
    return kivi_quantize(p, kind, max_tokens, static_cast<hipStream_t>(stream));
}

int eco_kivi_fake_quantize(void* buffer, int32_t format, int64_t sb, int64_t sh, int64_t ss, int32_t batch,
                           int32_t heads, int32_t slots, int32_t head_dim, int32_t start, int32_t stop, int32_t bits,
                           int32_t group, int32_t keys, void* stream) {
    if (!buffer) return fail("kivi fake quantize: null buffer");
    if (format != BF16 && format != FP16 && format != FP32)
        return fail("kivi fake quantize: the buffer must be bf16, fp16 or fp32");
    if (bits != 2 && bits != 4 && bits != 8) return fail("kivi fake quantize: bits must be 2, 4 or 8");
    if (batch < 0 || heads < 0 || head_dim <= 0 || group <= 0)
        return fail("kivi fake quantize: bad shape or group");
    if (start < 0 || stop < start || stop > slots) return fail("kivi fake quantize: slots out of the buffer");
    if (keys != 0 && keys != 1) return fail("kivi fake quantize: keys must be 0 or 1");
    if (keys && (stop - start) % group)
        return fail("kivi fake quantize: the key slots must be whole groups of tokens");
    if (!keys && head_dim % group) return fail("kivi fake quantize: the value group must divide the head dim");
    KiviFakeParams p{buffer, format, sb, sh, ss, batch, heads, head_dim, start, stop, bits, group, keys};
    return kivi_fake_quantize(p, static_cast<hipStream_t>(stream));
}

int eco_kivi_pack_quantize(int32_t kind, void* src, int32_t format, int64_t ss_b, int64_t ss_h, int64_t ss_s,
                           int32_t src_ring, int32_t write_back, void* codes, int64_t sc_b, int64_t sc_h, int64_t sc_s,
                           void* scale, void* zero, int64_t sz_b, int64_t sz_h, int64_t sz_s, const int32_t* from,
                           const int32_t* to, int32_t batch, int32_t heads, int32_t slots, int32_t head_dim,
                           int32_t bits, int32_t group, int32_t max_tokens, uint32_t* overflow, void* stream) {
    if (!src || !codes || !scale || !zero || !from || !to) return fail("kivi pack: null pointer");
    if (format != BF16 && format != FP16 && format != FP32)
        return fail("kivi pack: the source must be bf16, fp16 or fp32");
    if (bits != 2 && bits != 4 && bits != 8) return fail("kivi pack: bits must be 2, 4 or 8");
    if (kind != 0 && kind != 1) return fail("kivi pack: kind must be 0 (keys) or 1 (values)");
    if (batch < 0 || heads < 0 || slots < 0 || head_dim <= 0 || group <= 0 || max_tokens < 0 || src_ring < 0)
        return fail("kivi pack: bad shape, group or token count");
    if (head_dim % (8 / bits)) return fail("kivi pack: the head dim does not pack into whole bytes");
    if (kind == 0 && max_tokens % group) return fail("kivi pack: keys are quantized in whole groups of tokens");
    if (kind == 1 && head_dim % group) return fail("kivi pack: the value group must divide the head dim");
    if (write_back && src_ring) return fail("kivi pack: a ring source is not written back");
    KiviPackParams p{};
    p.src = src;
    p.format = format;
    p.ss_b = ss_b;
    p.ss_h = ss_h;
    p.ss_s = ss_s;
    p.src_ring = src_ring;
    p.write_back = write_back != 0;
    p.codes = static_cast<uint8_t*>(codes);
    p.sc_b = sc_b;
    p.sc_h = sc_h;
    p.sc_s = sc_s;
    p.scale = static_cast<uint16_t*>(scale);
    p.zero = static_cast<uint16_t*>(zero);
    p.sz_b = sz_b;
    p.sz_h = sz_h;
    p.sz_s = sz_s;
    p.from = from;
    p.to = to;
    p.batch = batch;
    p.heads = heads;
    p.head_dim = head_dim;
    p.bits = bits;
    p.group = group;
    p.max_tokens = max_tokens;
    p.keys = kind == 0;
    p.slots = slots;
    p.overflow = overflow;
    return kivi_pack_quantize(p, static_cast<hipStream_t>(stream));
}

int eco_kivi_packed_gather(int32_t kind, const uint8_t* codes, int64_t sc_b, int64_t sc_h, int64_t sc_s,
                           const void* scale, const void* zero, int64_t sz_b, int64_t sz_h, int64_t sz_s,
                           const int32_t* quantized, const void* ring, int64_t sr_b, int64_t sr_h, int64_t sr_s,
                           int32_t ring_slots, void* out, int32_t format, int64_t so_b, int64_t so_h, int64_t so_s,
                           int32_t batch, int32_t heads, int32_t slots, int32_t head_dim, int32_t bits, int32_t group,
                           void* stream) {
    if (!codes || !scale || !zero || !quantized || !ring || !out) return fail("kivi gather: null pointer");
    if (format != BF16 && format != FP16 && format != FP32)
        return fail("kivi gather: the ring and the output must be bf16, fp16 or fp32");
    if (bits != 2 && bits != 4 && bits != 8) return fail("kivi gather: bits must be 2, 4 or 8");
    if (kind != 0 && kind != 1) return fail("kivi gather: kind must be 0 (keys) or 1 (values)");
    if (batch < 0 || heads < 0 || slots < 0 || head_dim <= 0 || group <= 0 || ring_slots < 0)
        return fail("kivi gather: bad shape, group or ring");
    if (head_dim % (8 / bits) || (kind == 1 && head_dim % group))
        return fail("kivi gather: the head dim must pack into bytes (and hold whole value groups)");
    KiviRecordGatherParams p{};
    p.codes = codes;
    p.sc_b = sc_b;
    p.sc_h = sc_h;
    p.sc_s = sc_s;
    p.scale = static_cast<const uint16_t*>(scale);
    p.zero = static_cast<const uint16_t*>(zero);
    p.sz_b = sz_b;
    p.sz_h = sz_h;
    p.sz_s = sz_s;
    p.quantized = quantized;
    p.ring = ring;
    p.sr_b = sr_b;
    p.sr_h = sr_h;
    p.sr_s = sr_s;
    p.ring_slots = ring_slots;
    p.out = out;
    p.format = format;
    p.so_b = so_b;
    p.so_h = so_h;
    p.so_s = so_s;
    p.batch = batch;
    p.heads = heads;
    p.slots = slots;
    p.head_dim = head_dim;
    p.bits = bits;
    p.group = group;
    p.keys = kind == 0;
    return kivi_packed_gather(p, static_cast<hipStream_t>(stream));
}

int eco_kivi_cells_layout(int32_t head_dim, int32_t element_size, int32_t bits, int32_t group, int32_t* offsets) {
    if (!offsets) return fail("kivi cells layout: null output");
    CellLayout L;
    if (int rc = make_cell_layout(head_dim, element_size, bits, group, &L)) return rc;
    const int32_t values[10] = {L.value_group, L.key_aux, L.off_v, L.off_vs, L.off_vz,
                                L.off_ka,      L.off_kc,  L.off_vc, L.off_flag, L.size};
    std::memcpy(offsets, values, sizeof(values));
    return 0;
}

static int cells_params(void* cache, int32_t format, int64_t sb, int64_t sh, int64_t sn, int32_t num_pages,
                        int32_t page_size, int32_t kv_heads, int32_t head_dim, int32_t bits, int32_t group,
                        CellsParams* p) {
    if (!cache) return fail("kivi cells: null cache");
    if (format != BF16 && format != FP16 && format != FP32)
        return fail("kivi cells: the cache dtype must be bf16, fp16 or fp32");
    if (num_pages <= 0 || page_size <= 0 || kv_heads <= 0) return fail("kivi cells: pages and heads must be positive");
    std::memset(p, 0, sizeof(*p));
    if (int rc = make_cell_layout(head_dim, element_bytes(format), bits, group, &p->L)) return rc;
    if (page_size % group) return fail("kivi cells: pages must hold whole key groups");
    if (sn < p->L.size || sn % 16 || sh % 16 || sb % 16)
        return fail("kivi cells: cell strides must be multiples of 16 bytes, at least one cell");
    p->cache = static_cast<uint8_t*>(cache);
    p->sb = sb;
    p->sh = sh;
    p->sn = sn;
    p->format = format;
    p->page_size = page_size;
    p->num_pages = num_pages;
    p->kv_heads = kv_heads;
    return 0;
}

int eco_kivi_cells_quantize(void* cache, int32_t format, int64_t sb, int64_t sh, int64_t sn, int32_t num_pages,
                            int32_t page_size, int32_t kv_heads, const int32_t* block_table, int64_t bt_stride,
                            int32_t bt_cols, const int32_t* query_start_loc, const int32_t* seq_lens,
                            const int32_t* prefilling, int32_t requests, int32_t head_dim, int32_t bits,
                            int32_t group, int32_t residual, int32_t* plan, void* stream) {
    CellsParams p;
    if (int rc = cells_params(cache, format, sb, sh, sn, num_pages, page_size, kv_heads, head_dim, bits, group, &p))
        return rc;
    if (requests < 0) return fail("kivi cells quantize: negative request count");
    if (requests == 0) return 0;
    if (!block_table || !query_start_loc || !seq_lens || !prefilling || !plan)
        return fail("kivi cells quantize: null block table, query offsets, lengths, prefill flags or plan");
    if (bt_cols <= 0 || bt_stride < bt_cols) return fail("kivi cells quantize: bad block table");
    if (residual < group || residual % group) return fail("kivi cells quantize: the residual must be whole groups");
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.query_start_loc = query_start_loc;
    p.seq_lens = seq_lens;
    p.prefilling = prefilling;
    p.requests = requests;
    p.residual = residual;
    return kivi_cells_quantize(p, plan, static_cast<hipStream_t>(stream));
}

size_t eco_kivi_cells_attention_workspace_size(int32_t requests, int32_t max_query_len, int32_t q_heads,
                                               int32_t kv_heads, int32_t keys, int32_t head_dim) {
    if (requests <= 0 || max_query_len <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || keys < 0)
        return 0;
    if (!dense_padded_dim(head_dim, head_dim)) return 0;
    return dense_plan(requests, max_query_len, q_heads, kv_heads, std::max(keys, 1), head_dim, head_dim).workspace;
}

int eco_kivi_cells_attention(const void* q, int64_t sq_t, int64_t sq_h, const void* cache, int32_t format, int64_t sb,
                             int64_t sh, int64_t sn, int32_t num_pages, int32_t page_size, int32_t kv_heads,
                             const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                             const int32_t* query_start_loc, const int32_t* seq_lens, int32_t requests,
                             int32_t max_query_len, int32_t keys, int32_t head_dim, int32_t bits, int32_t group,
                             const float* sinks, void* out, int64_t so_t, int64_t so_h, int32_t q_heads, float scale,
                             float softcap, void* workspace, size_t workspace_bytes, void* stream) {
    CellsParams c;
    if (int rc = cells_params(const_cast<void*>(cache), format, sb, sh, sn, num_pages, page_size, kv_heads, head_dim,
                              bits, group, &c))
        return rc;
    if (!q || !out || !block_table || !query_start_loc || !seq_lens)
        return fail("kivi cells attention: null query, output, block table, query offsets or lengths");
    if (requests <= 0 || max_query_len <= 0 || q_heads <= 0 || keys <= 0)
        return fail("kivi cells attention: requests, max_query_len, query heads and keys must be positive");
    if (q_heads % kv_heads) return fail("kivi cells attention: query heads are not a multiple of the KV heads");
    if (bt_cols <= 0 || bt_stride < bt_cols) return fail("kivi cells attention: bad block table");
    if (page_size % 16) return fail("kivi cells attention: pages must hold a multiple of 16 tokens");
    const int es = element_bytes(format);
    if ((reinterpret_cast<uintptr_t>(q) & 15) || (sq_t * es) % 16 || (sq_h * es) % 16)
        return fail("kivi cells attention: the query must be 16-byte aligned with 16-byte strides");
    if (!(scale == scale)) return fail("kivi cells attention: scale is NaN");
    const DensePlan d = dense_plan(requests, max_query_len, q_heads, kv_heads, keys, head_dim, head_dim);
    if (!d.padded_dim) return fail("kivi cells attention: head dims up to 256");
    if (!workspace || workspace_bytes < d.workspace)
        return fail("kivi cells attention: workspace too small (" + std::to_string(workspace_bytes) + " < " +
                    std::to_string(d.workspace) + " bytes)");
    DenseParams p;
    std::memset(&p, 0, sizeof(p));
    p.q = q;
    p.sq_q = sq_t;
    p.sq_h = sq_h;
    p.q_format = format;
    p.k = cache;
    p.v = cache;
    p.kv_format = format;
    p.sinks = sinks;
    p.out = out;
    p.so_q = so_t;
    p.so_h = so_h;
    p.counters = static_cast<int32_t*>(workspace);
    p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + d.counter_bytes);
    p.batch = requests;
    p.queries = max_query_len;
    p.q_heads = q_heads;
    p.kv_heads = kv_heads;
    p.groups = q_heads / kv_heads;
    p.rows = p.groups * max_query_len;
    p.keys = keys;
    p.dense_keys = keys;
    p.head_dim = head_dim;
    p.value_dim = head_dim;
    p.m_tiles = d.m_tiles;
    p.splits = d.splits;
    p.scale = scale;
    p.softcap = softcap > 0.0f ? softcap : 0.0f;
    p.cells = static_cast<const uint8_t*>(cache);
    p.sc_page = sb;
    p.sc_head = sh;
    p.sc_token = sn;
    p.page_size = page_size;
    p.num_pages = num_pages;
    p.cell_off_v = c.L.off_v;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.seq_lens = seq_lens;
    p.query_start_loc = query_start_loc;
    p.causal = 1;
    // quantized cells through their codes (the reference's kernel reads them so) where the instance exists: bf16
    // cells of 128 channels, key groups of 32 (one 32-key tile is one group, whose 2 D scales and zero points sit in
    // the 8 aux slots of its 32 cells); otherwise every key and value from its dense entry, which quantize_committed
    // left holding the same dequantized numbers. ECO_CELLS_DENSE=1 forces the dense entries.
    static const bool force_dense = [] {
        const char* env = std::getenv("ECO_CELLS_DENSE");
        return env && env[0] == '1';
    }();
    if (format == BF16 && head_dim == 128 && group == 32 && c.L.key_aux == 8 && c.L.value_group == 32 &&
        (bits == 2 || bits == 4) && page_size % 32 == 0 && c.L.off_vz == c.L.off_vs + 8 && !force_dense) {
        p.code_bits = bits;
        p.cell_off_vs = c.L.off_vs;
        p.cell_off_ka = c.L.off_ka;
        p.cell_off_kc = c.L.off_kc;
        p.cell_off_vc = c.L.off_vc;
        p.cell_off_flag = c.L.off_flag;
    }
    return dense_attention(p, d.padded_dim, static_cast<hipStream_t>(stream));
}

int eco_kivi_cells_clear_flags(void* cache, int32_t format, int64_t sb, int64_t sh, int64_t sn, int32_t num_pages,
                               int32_t page_size, int32_t kv_heads, const int32_t* slots, int32_t tokens,
                               int32_t head_dim, int32_t bits, int32_t group, void* stream) {
    CellsParams p;
    if (int rc = cells_params(cache, format, sb, sh, sn, num_pages, page_size, kv_heads, head_dim, bits, group, &p))
        return rc;
    if (tokens < 0 || (tokens > 0 && !slots)) return fail("kivi cells clear: bad slots");
    return kivi_cells_clear_flags(p, slots, tokens, static_cast<hipStream_t>(stream));
}

int eco_kivi_ring_write(const void* k_new, const void* v_new, int32_t in_format, int64_t sk_t, int64_t sk_h,
                        int64_t sv_t, int64_t sv_h, const int32_t* rows, const int32_t* positions, int32_t tokens,
                        void* k_ring, void* v_ring, int32_t batch, int32_t kv_heads, int32_t head_dim, int32_t ring,
                        void* stream) {
    if (tokens < 0) return fail("kivi ring write: negative token count");
    if (tokens == 0) return 0;
    if (!k_new || !v_new || !rows || !positions || !k_ring || !v_ring) return fail("kivi ring write: null pointer");
    if (in_format != BF16 && in_format != FP16 && in_format != FP32)
        return fail("kivi ring write: inputs must be bf16, fp16 or fp32");
    if (batch <= 0 || kv_heads <= 0 || head_dim <= 0 || ring <= 0) return fail("kivi ring write: bad shape");
    KiviRingParams p{k_new, v_new, in_format, sk_t, sk_h, sv_t, sv_h, rows, positions, tokens,
                     static_cast<uint16_t*>(k_ring), static_cast<uint16_t*>(v_ring), batch, kv_heads, head_dim, ring};
    return kivi_ring_write(p, static_cast<hipStream_t>(stream));
}

size_t eco_kivi_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                                      int32_t head_dim, int32_t max_seq_len, int32_t bits) {
    if (batch <= 0 || queries <= 0 || kv_heads <= 0 || q_heads <= 0 || max_seq_len <= 0) return 0;
    if (check_kivi_shape(head_dim, bits, 32)) return 0;
    const int groups = q_heads / kv_heads;
    const QueryChunks qc = query_chunks(groups, queries);
    size_t need = 0;
    for (const int k : {qc.per, qc.last}) {
        const int grid = kivi_grid(batch, kv_heads, groups * k, head_dim, bits, max_seq_len);
        if (grid <= 0) return 0;
        need = std::max(need, paged_workspace(batch, kv_heads, groups * k, head_dim, grid).total());
    }
    return need;
}

int eco_kivi_decode(const void* q, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* blocks, int32_t num_pages,
                    const void* k_ring, const void* v_ring, int32_t ring, const int32_t* keys_quantized,
                    const int32_t* values_quantized, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                    const int32_t* seq_lens, const float* sinks, void* out, int64_t so_b, int64_t so_q, int64_t so_h,
                    int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                    int32_t bits, int32_t group, int32_t max_seq_len, float scale, float softcap,
                    const uint32_t* mask_bits, int64_t mk_b, int64_t mk_h, int64_t mk_q, int32_t mask_words,
                    void* workspace, size_t workspace_bytes, void* stream) {
    if (!q || !blocks || !k_ring || !v_ring || !keys_quantized || !values_quantized || !block_table || !seq_lens ||
        !out)
        return fail("kivi decode: null query, cache, ring, counts, table, lengths or output");
    if (batch <= 0 || queries <= 0 || q_heads <= 0 || kv_heads <= 0 || num_pages <= 0 || bt_cols <= 0 ||
        bt_stride < bt_cols)
        return fail("kivi decode: batch, queries, heads, pages and block-table columns must be positive");
    if (q_heads % kv_heads) return fail("kivi decode: query heads are not a multiple of the KV heads");
    if (int rc = check_kivi_shape(head_dim, bits, group)) return rc;
    if (ring <= 0 || ring % 32) return fail("kivi decode: the ring must hold a positive multiple of 32 slots");
    const int groups = q_heads / kv_heads;
    if (groups > 64) return fail("kivi decode: at most 64 query heads per KV head");
    const QueryChunks qc = query_chunks(groups, queries);
    if ((reinterpret_cast<uintptr_t>(q) & 15) || (sq_b & 7) || (sq_q & 7) || (sq_h & 7))
        return fail("kivi decode: the query must be 16-byte aligned with strides that are multiples of 8");
    if (max_seq_len <= 0) return fail("kivi decode: max_seq_len must be positive");
    if (!(scale == scale)) return fail("kivi decode: scale is NaN");
    if (mask_bits && mask_words <= 0) return fail("kivi decode: a mask needs a positive word count");
    // the launch plan of each chunk shape (every chunk but the last, then the last)
    int grids[2];
    size_t need = 0;
    for (int i = 0; i < 2; ++i) {
        const int rows_i = groups * (i == 0 ? qc.per : qc.last);
        grids[i] = kivi_grid(batch, kv_heads, rows_i, head_dim, bits, max_seq_len);
        if (grids[i] <= 0) return 1;
        need = std::max(need, paged_workspace(batch, kv_heads, rows_i, head_dim, grids[i]).total());
    }
    if (!workspace || workspace_bytes < need)
        return fail("kivi decode: workspace too small (" + std::to_string(workspace_bytes) + " < " +
                    std::to_string(need) + " bytes)");
    const KiviLayout L{head_dim, bits};
    KiviParams p;
    std::memset(&p, 0, sizeof(p));
    p.q = static_cast<const uint16_t*>(q);
    p.sq_b = sq_b;
    p.sq_q = sq_q;
    p.sq_h = sq_h;
    p.blocks = static_cast<const uint8_t*>(blocks);
    p.blk_head = L.size();
    p.blk_page = static_cast<int64_t>(L.size()) * kv_heads;
    p.k_ring = static_cast<const uint16_t*>(k_ring);
    p.v_ring = static_cast<const uint16_t*>(v_ring);
    p.ring = ring;
    p.keys_quantized = keys_quantized;
    p.values_quantized = values_quantized;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.num_pages = num_pages;
    p.seq_lens = seq_lens;
    p.sinks = sinks;
    p.mask = mask_bits;
    p.mk_b = mk_b;
    p.mk_h = mk_h;
    p.mk_q = mk_q;
    p.mask_words = mask_bits ? mask_words : 0;
    char* base = static_cast<char*>(workspace);
    p.counters = reinterpret_cast<int32_t*>(base);
    p.part = reinterpret_cast<float*>(base + paged_workspace(batch, kv_heads, 1, head_dim, 1).counter_bytes);
    p.so_b = so_b;
    p.so_q = so_q;
    p.so_h = so_h;
    p.batch = batch;
    p.q_heads = q_heads;
    p.kv_heads = kv_heads;
    p.groups = groups;
    p.head_dim = head_dim;
    p.bits = bits;
    p.scale = scale;
    p.softcap = softcap > 0.0f ? softcap : 0.0f;
    for (int c = 0; c < qc.count; ++c) {
        const int q0 = c * qc.per, k = c + 1 < qc.count ? qc.per : qc.last;
        p.q = static_cast<const uint16_t*>(q) + q0 * sq_q;
        p.out = static_cast<uint16_t*>(out) + q0 * so_q;
        p.mask = mask_bits ? mask_bits + q0 * mk_q : nullptr;
        p.queries = k;
        p.queries_after = queries - q0 - k;
        p.rows = groups * k;
        p.grid = grids[c + 1 < qc.count ? 0 : 1];
        if (const int rc = kivi_attention(p, static_cast<hipStream_t>(stream))) return rc;
    }
    return 0;
}

int eco_quest_page_bounds(const void* k_cache, int32_t kv_format, int32_t num_pages, const int32_t* block_table,
                          int64_t bt_stride, int32_t bt_cols, int32_t first, int32_t last, int32_t quest_page_size,
                          void* kmin, void* kmax, int64_t sb_b, int64_t sb_h, int64_t sb_p, int32_t batch,
                          int32_t kv_heads, int32_t head_dim, int32_t page_size, void* stream) {
    if (!k_cache || !block_table || !kmin || !kmax) return fail("quest page bounds: null cache, table or bounds");
    if (batch <= 0 || kv_heads <= 0 || num_pages <= 0 || bt_cols <= 0 || bt_stride < bt_cols)
        return fail("quest page bounds: batch, heads, pages and block-table columns must be positive");
    if (page_size != 16) return fail("quest page bounds: cache pages must hold 16 tokens");
    if (quest_page_size < 16 || quest_page_size % 16 || (quest_page_size & (quest_page_size - 1)))
        return fail("quest page bounds: quest pages must hold a power of two of at least 16 tokens");
    if (kv_format != BF16 && kv_format != FP8_E4M3 && kv_format != FP8_E5M2)
        return fail("quest page bounds: KV format must be bf16, fp8 e4m3 or fp8 e5m2");
    const int es = kv_format == BF16 ? 2 : 1;
    if (head_dim <= 0 || (head_dim * es) % 64) return fail("quest page bounds: head dim must fill whole runs");
    if (first < 0 || last < first) return fail("quest page bounds: need 0 <= first <= last");
    BoundsParams p;
    p.k_cache = static_cast<const uint8_t*>(k_cache);
    p.kc_head = static_cast<int64_t>(head_dim) * 16 * es;
    p.kc_page = p.kc_head * kv_heads;
    p.kv_format = kv_format;
    p.num_pages = num_pages;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.first = first;
    p.last = last;
    p.span = quest_page_size / 16;
    p.kmin = static_cast<uint16_t*>(kmin);
    p.kmax = static_cast<uint16_t*>(kmax);
    p.sb_b = sb_b;
    p.sb_h = sb_h;
    p.sb_p = sb_p;
    p.batch = batch;
    p.kv_heads = kv_heads;
    p.head_dim = head_dim;
    p.committed = nullptr;
    p.valid = nullptr;
    p.done = nullptr;
    p.page_cap = 0;
    return quest_bounds(p, static_cast<hipStream_t>(stream));
}

int eco_quest_refresh_bounds(const void* k_cache, int32_t kv_format, int32_t num_pages, const int32_t* block_table,
                             int64_t bt_stride, int32_t bt_cols, const int32_t* committed, int32_t* valid,
                             int32_t* done, int32_t quest_page_size, void* kmin, void* kmax, int64_t sb_b,
                             int64_t sb_h, int64_t sb_p, int32_t page_cap, int32_t batch, int32_t kv_heads,
                             int32_t head_dim, int32_t page_size, void* stream) {
    if (!k_cache || !block_table || !kmin || !kmax || !committed || !valid)
        return fail("quest refresh: null cache, table, bounds, committed or valid");
    if (batch <= 0 || kv_heads <= 0 || num_pages <= 0 || bt_cols <= 0 || bt_stride < bt_cols || page_cap < 0)
        return fail("quest refresh: batch, heads, pages and block-table columns must be positive");
    if (page_size != 16) return fail("quest refresh: cache pages must hold 16 tokens");
    if (quest_page_size < 16 || quest_page_size % 16 || (quest_page_size & (quest_page_size - 1)))
        return fail("quest refresh: quest pages must hold a power of two of at least 16 tokens");
    if (kv_format != BF16 && kv_format != FP8_E4M3 && kv_format != FP8_E5M2)
        return fail("quest refresh: KV format must be bf16, fp8 e4m3 or fp8 e5m2");
    const int es = kv_format == BF16 ? 2 : 1;
    if (head_dim <= 0 || (head_dim * es) % 64) return fail("quest refresh: head dim must fill whole runs");
    BoundsParams p;
    p.k_cache = static_cast<const uint8_t*>(k_cache);
    p.kc_head = static_cast<int64_t>(head_dim) * 16 * es;
    p.kc_page = p.kc_head * kv_heads;
    p.kv_format = kv_format;
    p.num_pages = num_pages;
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.bt_cols = bt_cols;
    p.first = 0;
    p.last = 0;
    p.span = quest_page_size / 16;
    p.kmin = static_cast<uint16_t*>(kmin);
    p.kmax = static_cast<uint16_t*>(kmax);
    p.sb_b = sb_b;
    p.sb_h = sb_h;
    p.sb_p = sb_p;
    p.batch = batch;
    p.kv_heads = kv_heads;
    p.head_dim = head_dim;
    p.committed = committed;
    p.valid = valid;
    p.done = done;
    p.page_cap = page_cap;
    return quest_refresh(p, static_cast<hipStream_t>(stream));
}

int eco_quest_dense_bounds(const void* keys, int32_t kv_format, int64_t sk_b, int64_t sk_h, int64_t sk_s,
                           int32_t slots, int32_t first, int32_t last, int32_t page_size, void* kmin, void* kmax,
                           int32_t bounds_format, int64_t sb_b, int64_t sb_h, int64_t sb_p, int32_t batch,
                           int32_t kv_heads, int32_t head_dim, void* stream) {
    if (!keys || !kmin || !kmax) return fail("quest page bounds: null keys or bounds");
    if (batch <= 0 || kv_heads <= 0 || head_dim <= 0 || slots < 0)
        return fail("quest page bounds: batch, heads and head dim must be positive, slots non-negative");
    if (page_size < 16 || (page_size & (page_size - 1)))
        return fail("quest page bounds: pages must hold a power of two of at least 16 slots");
    if (first < 0 || last < first || static_cast<int64_t>(last) * page_size > slots)
        return fail("quest page bounds: need 0 <= first <= last and last pages within the " + std::to_string(slots) +
                    " slots");
    const bool fp8 = kv_format == FP8_E4M3 || kv_format == FP8_E5M2;
    if (kv_format != BF16 && kv_format != FP16 && kv_format != FP32 && !fp8)
        return fail("quest page bounds: keys must be bf16, fp16, fp32, fp8 e4m3 or fp8 e5m2");
    const int want = fp8 ? BF16 : kv_format;  // bounds_dtype (attention/quest.py:68-70)
    if (bounds_format != want) return fail("quest page bounds: bounds must be bf16 for bf16 and fp8 keys, else the keys' dtype");
    DenseBoundsParams p;
    p.keys = keys;
    p.sk_b = sk_b;
    p.sk_h = sk_h;
    p.sk_s = sk_s;
    p.kv_format = kv_format;
    p.first = first;
    p.last = last;
    p.page = page_size;
    p.kmin = kmin;
    p.kmax = kmax;
    p.sb_b = sb_b;
    p.sb_h = sb_h;
    p.sb_p = sb_p;
    p.bounds_format = bounds_format;
    p.batch = batch;
    p.kv_heads = kv_heads;
    p.head_dim = head_dim;
    return quest_dense_bounds(p, static_cast<hipStream_t>(stream));
}

int eco_quest_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
                     const void* v, int32_t kv_format, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b,
                     int64_t sv_h, int64_t sv_s, const float* k_scale, const float* v_scale, const int32_t* index,
                     int64_t si_b, int64_t si_h, int32_t pages, const int32_t* done, int32_t page_size,
                     int32_t min_done, const uint8_t* mask, int64_t sm_b, int64_t sm_h, int64_t sm_q, int64_t sm_s,
                     const float* sinks, void* out, int64_t so_b, int64_t so_q, int64_t so_h, int32_t batch,
                     int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys, int32_t head_dim,
                     int32_t value_dim, float scale, float softcap, void* workspace, size_t workspace_bytes,
                     void* stream) {
    if (!index || !done) return fail("quest decode: null page index or done");
    if (page_size < 16 || (page_size & (page_size - 1)))
        return fail("quest decode: pages must hold a power of two of at least 16 slots");
    if (pages < 0 || min_done < 0 || static_cast<int64_t>(min_done) * page_size > keys)
        return fail("quest decode: need pages >= 0 and 0 <= min_done * page <= keys");
    int shift = 0;
    while ((1 << shift) < page_size) ++shift;
    const QuestListArgs ql{index, si_b, si_h, pages, shift, min_done, done};
    return dense_decode(q, q_format, sq_b, sq_h, sq_q, k, v, kv_format, sk_b, sk_h, sk_s, sv_b, sv_h, sv_s, k_scale,
                        v_scale, mask, sm_b, sm_h, sm_q, sm_s, sinks, out, so_b, so_q, so_h, batch, queries, q_heads,
                        kv_heads, keys, head_dim, value_dim, scale, softcap, workspace, workspace_bytes, stream,
                        nullptr, &ql);
}

size_t eco_quest_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                                       int32_t keys, int32_t pages, int32_t page_size, int32_t min_done,
                                       int32_t head_dim, int32_t value_dim) {
    if (page_size < 16 || pages < 0 || min_done < 0) return 0;
    const int64_t virt = std::max<int64_t>(1, static_cast<int64_t>(pages) * page_size + keys -
                                                  static_cast<int64_t>(min_done) * page_size);
    if (virt > INT32_MAX) return 0;
    return eco_decode_workspace_size(batch, queries, q_heads, kv_heads, static_cast<int32_t>(virt), head_dim,
                                     value_dim);
}

int eco_kivi_packed_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
                           const void* v, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b, int64_t sv_h,
                           int64_t sv_s, int32_t ring, const uint8_t* key_codes, int64_t skc_b, int64_t skc_h,
                           int64_t skc_s, const void* key_scale, const void* key_zero, int64_t sks_b, int64_t sks_h,
                           int64_t sks_g, const uint8_t* value_codes, int64_t svc_b, int64_t svc_h, int64_t svc_s,
                           const void* value_scale, const void* value_zero, int64_t svs_b, int64_t svs_h,
                           int64_t svs_s, const int32_t* keys_quantized, const int32_t* values_quantized,
                           int32_t bits, int32_t key_group, int32_t value_group, const uint8_t* mask, int64_t sm_b,
                           int64_t sm_h, int64_t sm_q, int64_t sm_s, const float* sinks, void* out, int64_t so_b,
                           int64_t so_q, int64_t so_h, int32_t batch, int32_t queries, int32_t q_heads,
                           int32_t kv_heads, int32_t keys, int32_t head_dim, int32_t value_dim, float scale,
                           float softcap, void* workspace, size_t workspace_bytes, void* stream) {
    if (!key_codes || !key_scale || !key_zero || !value_codes || !value_scale || !value_zero)
        return fail("kivi decode: null codes, scales or zero points");
    if (!keys_quantized || !values_quantized) return fail("kivi decode: null quantized counts");
    if (bits != 2 && bits != 4 && bits != 8) return fail("kivi decode: bits must be 2, 4 or 8");
    if (keys <= 0) return fail("kivi decode: need keys > 0");
    if (ring < 0) return fail("kivi decode: ring must be non-negative");
    if (key_group <= 0 || value_group <= 0 || value_dim <= 0 || value_dim % value_group)
        return fail("kivi decode: the value group must divide the value head dim (groups positive)");
    if (q_format != BF16 && q_format != FP16 && q_format != FP32)
        return fail("kivi decode: queries must be bf16, fp16 or fp32");
    const int ce = 16 / element_bytes(q_format);  // elements per 16-byte chunk of the kernel
    const int nb = ce * bits / 8;                  // code bytes of a chunk
    auto aligned_to = [](const void* ptr, int bytes) { return (reinterpret_cast<uintptr_t>(ptr) % bytes) == 0; };
    if (!aligned_to(key_codes, nb) || !aligned_to(value_codes, nb))
        return fail("kivi decode: codes must be aligned to " + std::to_string(nb) + " bytes");
    for (int64_t st : {skc_b, skc_h, skc_s, svc_b, svc_h, svc_s})
        if (st % nb) return fail("kivi decode: code strides must be multiples of " + std::to_string(nb) + " bytes");
    if (!aligned_to(key_scale, 2 * ce) || !aligned_to(key_zero, 2 * ce))
        return fail("kivi decode: key scales and zero points must be aligned to " + std::to_string(2 * ce) + " bytes");
    for (int64_t st : {sks_b, sks_h, sks_g})
        if (st % ce) return fail("kivi decode: key scale strides must be multiples of " + std::to_string(ce) + " elements");
    if (!aligned_to(value_scale, 2) || !aligned_to(value_zero, 2))
        return fail("kivi decode: value scales and zero points must be fp16-aligned");
    const KiviPackedArgs kp{key_codes, skc_b, skc_h, skc_s, static_cast<const uint16_t*>(key_scale),
                            static_cast<const uint16_t*>(key_zero), sks_b, sks_h, sks_g, value_codes, svc_b, svc_h,
                            svc_s, static_cast<const uint16_t*>(value_scale), static_cast<const uint16_t*>(value_zero),
                            svs_b, svs_h, svs_s, keys_quantized, values_quantized, bits, key_group, value_group, ring};
    return dense_decode(q, q_format, sq_b, sq_h, sq_q, k, v, q_format, sk_b, sk_h, sk_s, sv_b, sv_h, sv_s, nullptr,
                        nullptr, mask, sm_b, sm_h, sm_q, sm_s, sinks, out, so_b, so_q, so_h, batch, queries, q_heads,
                        kv_heads, keys, head_dim, value_dim, scale, softcap, workspace, workspace_bytes, stream,
                        nullptr, nullptr, &kp);
}

size_t eco_quest_select_workspace_size(int32_t batch, int32_t kv_heads, int32_t max_done) {
    if (batch <= 0 || kv_heads <= 0 || max_done < 0) return 0;
    const size_t stride = (static_cast<size_t>(max_done > 0 ? max_done : 1) + 3) / 4 * 4;  // 16-byte aligned rows
    return align256(static_cast<size_t>(batch) * kv_heads * stride * sizeof(float));
}

int eco_quest_select(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* kmin,
                     const void* kmax, int32_t bounds_format, int64_t sb_b, int64_t sb_h, int64_t sb_p,
                     const int32_t* done, int32_t max_done, int32_t pages, int32_t first_page, int32_t* out,
                     int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                     void* workspace, size_t workspace_bytes, void* stream) {
    if (!q || !done || !out) return fail("quest select: null query, done or output");
    for (int f : {q_format, bounds_format})
        if (f != BF16 && f != FP16 && f != FP32) return fail("quest select: queries and bounds must be bf16, fp16 or fp32");
    if (batch <= 0 || queries <= 0 || q_heads <= 0 || kv_heads <= 0 || pages < 0 || max_done < 0)
        return fail("quest select: batch, queries and heads must be positive, pages and max_done non-negative");
    if (q_heads % kv_heads) return fail("quest select: query heads are not a multiple of the KV heads");
    if (head_dim <= 0 || head_dim % 8 || head_dim > 512) return fail("quest select: head dim must be a multiple of 8 up to 512");
    if (max_done > 0 && (!kmin || !kmax)) return fail("quest select: null page bounds");
    if ((reinterpret_cast<uintptr_t>(kmin) & 15) || (reinterpret_cast<uintptr_t>(kmax) & 15) || (sb_b & 7) ||
        (sb_h & 7) || (sb_p & 7))
        return fail("quest select: page bounds must be 16-byte aligned with strides that are multiples of 8 elements");
    if (pages == 0) return 0;
    const size_t need = eco_quest_select_workspace_size(batch, kv_heads, max_done);
    if (max_done > 0 && (!workspace || workspace_bytes < need))
        return fail("quest select: workspace too small (" + std::to_string(workspace_bytes) + " < " +
                    std::to_string(need) + " bytes)");
    SelectParams p;
    p.q = q;
    p.q_format = q_format;
    p.sq_b = sq_b;
    p.sq_q = sq_q;
    p.sq_h = sq_h;
    p.kmin = kmin;
    p.kmax = kmax;
    p.bounds_format = bounds_format;
    p.sb_b = sb_b;
    p.sb_h = sb_h;
    p.sb_p = sb_p;
    p.done = done;
    p.max_done = max_done;
    p.pages = pages;
    p.first_page = first_page != 0;
    p.out = out;
    p.scores = static_cast<float*>(workspace);
    p.batch = batch;
    p.queries = queries;
    p.q_heads = q_heads;
    p.kv_heads = kv_heads;
    p.groups = q_heads / kv_heads;
    p.head_dim = head_dim;
    p.chunk = quest_score_chunk(head_dim);
    return quest_select(p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
