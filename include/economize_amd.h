/* economize_amd: C ABI of the compressed-KV decode-attention kernels for AMD MI355X (gfx950).
 *
 * Every entry point takes plain device pointers, sizes and strides, launches asynchronously on the given HIP
 * stream (hipStream_t passed as void*; NULL = the null stream) and returns 0, or nonzero with a message that
 * eco_last_error() returns (validation errors are raised before any launch, as the reference raises ConfigError
 * before launching, attention/decode.py:287-300). Nothing allocates device memory: scratch space is a caller-owned
 * workspace whose size the matching *_workspace_size function returns.
 *
 * Element formats: ECO_BF16, ECO_FP8_E4M3 (OCP e4m3fn), ECO_FP8_E5M2, ECO_FP16, ECO_FP32.
 *
 * Paged KV cache (16-token pages, vLLM's paged-attention layout), per layer:
 *   keys   [num_pages, Hkv, D / X, 16, X]  X = 16 / element bytes
 *   values [num_pages, Hkv, D, 16]
 * Row b's token t lives in page block_table[b * bt_stride + t / 16] at position t % 16 (t / 16 < bt_cols).
 * Kernels skip table entries outside [0, num_pages) and logical pages outside [0, bt_cols), so a malformed table
 * reads nothing out of bounds (it gives wrong results instead).
 */
#ifndef ECONOMIZE_AMD_H
#define ECONOMIZE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ECO_BF16 = 0, ECO_FP8_E4M3 = 1, ECO_FP8_E5M2 = 2, ECO_FP16 = 3, ECO_FP32 = 4 };

/* The message of the last failed call on this thread ("" if none). */
const char* eco_last_error(void);

/* Version of this ABI (bumped on incompatible changes). */
int eco_abi_version(void);

/* FP8 / bf16 quantize-and-append into the paged cache.
 * Replaces the reference's FP8Cache.transform_update + fp8_encode + write_slots
 * (techniques/kv_quant/fp8.py:81-86, 161-176; modules/kv_cache.py:30-41): k_new / v_new [tokens, Hkv, D] (channel
 * stride 1, element strides sk_t, sk_h, sv_t, sv_h, format in_format = bf16, fp16 or fp32) are divided by the
 * per-head scale (k_scale / v_scale [Hkv] fp32, or NULL for none), clamped to the format's maximum, rounded to
 * nearest even and stored at slot_mapping[t] (slot = page * 16 + position; negative = skip). A bf16 cache stores the
 * values rounded to bf16. */
int eco_paged_append(const void* k_new, const void* v_new, int32_t in_format, int64_t sk_t, int64_t sk_h,
                     int64_t sv_t, int64_t sv_h, const int32_t* slot_mapping, int32_t tokens, void* k_cache,
                     void* v_cache, int32_t num_pages, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                     int32_t cache_format, const float* k_scale, const float* v_scale, void* stream);

/* eco_paged_append plus Quest's page bounds kept on the device, in one launch: the new tokens are appended as
 * eco_paged_append does, and the bounds of the Quest pages each row b and KV head h committed since the last call
 * (pages [valid[b * Hkv + h], min(committed[b] / quest_page_size, page_cap))) are computed as
 * eco_quest_refresh_bounds does, after which valid advances and done[b] (optional) becomes the row's committed Quest
 * pages. counters (int32 [B * Hkv]) must be zero before the first call; every call leaves them zero. The appended
 * tokens must lie at or past the committed ones (the launch refreshes pages it does not write). tokens may be 0 (a
 * refresh only). The launch shape depends on the arguments only, so a decode step can be captured in a graph.
 * Replaces FP8Cache.transform_update (techniques/kv_quant/fp8.py:161-176) together with QuestCache.pass_begin and
 * _layer_bounds (techniques/quest/technique.py:165-172, 229-259), whose host done list keeps the reference's Quest
 * out of graphs (technique.py:311). */
int eco_paged_append_quest(const void* k_new, const void* v_new, int32_t in_format, int64_t sk_t, int64_t sk_h,
                           int64_t sv_t, int64_t sv_h, const int32_t* slot_mapping, int32_t tokens, void* k_cache,
                           void* v_cache, int32_t num_pages, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                           int32_t cache_format, const float* k_scale, const float* v_scale,
                           const int32_t* block_table, int64_t bt_stride, int32_t bt_cols, const int32_t* committed,
                           int32_t* valid, int32_t* done, int32_t* counters, int32_t quest_page_size, void* kmin,
                           void* kmax, int64_t sb_b, int64_t sb_h, int64_t sb_p, int32_t page_cap, int32_t batch,
                           void* stream);

/* fp8 encode into a dense fp8 buffer (the fused fp8 cache's [B, H, S, D] buffers).
 * Replaces the reference's fp8_encode and token_scale (techniques/kv_quant/fp8.py:81-86, 95-97) as
 * FP8Cache.transform_update applies them (fp8.py:161-176): src [B, H, T, D] (element strides ss_b, ss_h, ss_t,
 * channel stride 1, bf16 / fp16 / fp32) is divided by its scale, clamped to the format's maximum, rounded to nearest
 * even and written to dst (byte strides sd_b, sd_h, sd_t, channel stride 1). Scales: head_scale [H] fp32 (the static
 * and per-head modes), or token_scale non-NULL (the per-token mode: each (b, h, t) row's absmax / format max, at
 * least 1e-12, written to token_scale at element strides st_b, st_h, st_t), or neither (a direct cast). */
int eco_fp8_encode(const void* src, int32_t in_format, int64_t ss_b, int64_t ss_h, int64_t ss_t, void* dst,
                   int32_t out_format, int64_t sd_b, int64_t sd_h, int64_t sd_t, int32_t batch, int32_t heads,
                   int32_t tokens, int32_t head_dim, const float* head_scale, float* token_scale, int64_t st_b,
                   int64_t st_h, int64_t st_t, void* stream);

/* Per-head absolute maximum of x [A, H, S, D] (element strides sa, sh, ss, sd; format bf16, fp16 or fp32),
 * max-accumulated into absmax_bits[H] as float bit patterns (zero them before the first call). With
 * eco_fp8_scales_from_absmax it is the reference's calibrate_kv_absmax + static_scales
 * (techniques/kv_quant/fp8.py:100-133) per KV head. */
int eco_kv_head_absmax(const void* x, int32_t in_format, int32_t a, int32_t h, int32_t s, int32_t d, int64_t sa,
                       int64_t sh, int64_t ss, int64_t sd, uint32_t* absmax_bits, void* stream);

/* scales[h] = absmax[h] / format max (IEEE division), 1 where that is not positive (fp8.py:130-133). */
int eco_fp8_scales_from_absmax(const uint32_t* absmax_bits, int32_t heads, int32_t format, float* scales,
                               void* stream);

/* Workspace bytes eco_paged_decode needs for this shape (n_sel = Quest's selected pages of list_page_size tokens,
 * 0 without). The workspace starts with per-row counters, int32 per batch row and KV head, padded to 256 bytes,
 * which must be zero when a call starts; every call leaves them zero and may write anything after them, so a call
 * with more rows times KV heads than the previous one on the same workspace needs the bytes between cleared first.
 * One workspace serves one stream at a time. */
size_t eco_paged_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                                       int32_t head_dim, int32_t max_seq_len, int32_t n_sel, int32_t list_page_size,
                                       int32_t kv_format);

/* Split-K decode attention over the paged cache: out[b, qi, h, :] (element strides so_*, the query's format) for
 * query q[b, qi, h, :] (q_format bf16, or fp16 with an fp8 cache and no page list: a model in fp16; element strides
 * sq_*, channel stride 1), query head h reading KV head h / (q_heads / kv_heads).
 * Row b holds seq_lens[b] tokens, its queries the last `queries` of them, query qi seeing tokens
 * < seq_lens[b] - queries + qi + 1. Scores are q . k * scale (k, v decoded times k_scale / v_scale [Hkv], NULL =
 * 1), an optional softcap > 0 applies softcap * tanh(s / softcap), optional sinks [Hq] join the softmax's
 * denominator. A row that sees no key gives 0.
 * Replaces decode_attention (attention/decode.py:252-324) for a paged cache, and with page_list != NULL
 * quest_decode_attention (attention/quest.py:239-344): the keys read are the pages page_list[b, kvh, 0..n_sel)
 * (strides pl_b, pl_h; page indices of list_page_size tokens each, 0 = 16; pages below done[b] are read, others
 * read nothing) and then every token from page done[b] on (done in listed pages too). One launch: the work is cut
 * into equal contiguous ranges of 64-token tiles, one per wave, so ragged rows need no host-side plan; max_seq_len
 * (>= every seq_lens[b]) only bounds the launch. An optional packed attention mask (eco_mask_bits: bit t % 32 of word
 * mask_bits[b * mk_b + h * mk_h + qi * mk_q + t / 32], word strides 0 on broadcast axes, mask_words words per row;
 * NULL = none) hides token t from query qi of head h where its bit is 0, on top of the causal limit. At most 64
 * query heads per KV head; a call of more than 64 query rows per KV head (query heads per KV head x queries) runs as
 * consecutive launches over chunks of floor(64 / (q_heads / kv_heads)) queries on the stream. */
int eco_paged_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* k_cache,
                     const void* v_cache, int32_t kv_format, int32_t num_pages, const float* k_scale,
                     const float* v_scale, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                     const int32_t* seq_lens, const int32_t* page_list, int64_t pl_b, int64_t pl_h, int32_t n_sel,
                     int32_t list_page_size, const int32_t* done, const float* sinks, void* out, int64_t so_b,
                     int64_t so_q, int64_t so_h, int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                     int32_t head_dim, int32_t page_size, int32_t max_seq_len, float scale, float softcap,
                     const uint32_t* mask_bits, int64_t mk_b, int64_t mk_h, int64_t mk_q, int32_t mask_words,
                     void* workspace, size_t workspace_bytes, void* stream);

/* eco_paged_decode (bf16 queries) without a workspace: the scratch is the library's own, so the call allocates nothing
 * (neither the library nor the caller). No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The scratch is one static
 * device array of 32 MiB per GPU, held until the process ends; a call whose workspace
 * (eco_paged_decode_workspace_size) would be larger is refused before any launch. Each call clears the array's row
 * counters with a fill kernel on its stream before the attention kernel. Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (on other streams or host threads) race. */
int eco_paged_decode_static(const void* q, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* k_cache,
                            const void* v_cache, int32_t kv_format, int32_t num_pages, const float* k_scale,
                            const float* v_scale, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                            const int32_t* seq_lens, const int32_t* page_list, int64_t pl_b, int64_t pl_h,
                            int32_t n_sel, int32_t list_page_size, const int32_t* done, const float* sinks, void* out,
                            int64_t so_b, int64_t so_q, int64_t so_h, int32_t batch, int32_t queries,
                            int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                            int32_t max_seq_len, float scale, float softcap, const uint32_t* mask_bits, int64_t mk_b,
                            int64_t mk_h, int64_t mk_q, int32_t mask_words, void* stream);

/* Decode attention over a cache whose prompt entries were compacted by an eviction (the reference's
 * gathered_decode_attention and GatheredKV, attention/gathered.py:39-179): for row b and KV head h, virtual key t is
 * compact entry t of ck / cv [B, Hkv, capacity, D / Dv] (strides sck_*, scv_*; mask column index[b, h, t], strides
 * si_b, si_h) below count[b * Hkv + h], else dense slot start[b] + t - count of k / v [B, Hkv, keys, D / Dv]; the
 * virtual axis is keys - dropped long (dropped = min(start[b] - count[b, h]) on the host). Everything else as
 * eco_decode, with K/V in the query's format; the workspace is eco_decode_workspace_size(..., keys - dropped, ...)
 * bytes under eco_decode's counter rule.
 * Counts beyond the capacity and starts beyond the slots are clamped (wrong results, no access outside a buffer). */
int eco_gathered_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
                        const void* v, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b, int64_t sv_h,
                        int64_t sv_s, const void* ck, const void* cv, int64_t sck_b, int64_t sck_h, int64_t sck_s,
                        int64_t scv_b, int64_t scv_h, int64_t scv_s, const int32_t* index, int64_t si_b,
                        int64_t si_h, const int32_t* count, const int32_t* start, int32_t capacity, int32_t dropped,
                        const uint8_t* mask, int64_t sm_b, int64_t sm_h, int64_t sm_q, int64_t sm_s,
                        const float* sinks, void* out, int64_t so_b, int64_t so_q, int64_t so_h, int32_t batch,
                        int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys, int32_t head_dim,
                        int32_t value_dim, float scale, float softcap, void* workspace, size_t workspace_bytes,
                        void* stream);

/* The packed form of a boolean attention mask that the paged decode kernels take: bits[((b * heads + h) * queries +
 * q) * words + w] has bit k set where mask[b * sm_b + h * sm_h + q * sm_q + (32 w + k) * sm_s] is nonzero (one byte
 * per element; 0 past `keys`). words >= ceil(keys / 32). A broadcast axis of the mask is packed once (pass its size
 * as 1) and read through a word stride of 0. No counterpart in the reference, whose kernels read the bytes
 * (attention/_decode_kernels.py:67-74); a packed word per 32 keys is one aligned load per tile here. */
int eco_mask_bits(const uint8_t* mask, int64_t sm_b, int64_t sm_h, int64_t sm_q, int64_t sm_s, int32_t batch,
                  int32_t heads, int32_t queries, int32_t keys, uint32_t* bits, int32_t words, void* stream);

/* The dense view of the paged fp8 / bf16 cache: k_out / v_out [b, kvh, t, :] (element strides so_k*, so_v*; format
 * out_format = bf16, fp16 or fp32) = the stored keys and values of tokens t < keys, fp8 decoded exactly and times
 * the per-head scales (NULL = 1), 0 for tokens past a row's table. Replaces materialize() of a cache without dense
 * buffers (attention/packed.py:66-78) for the attention functions that do not read the paged format. */
int eco_paged_gather(const void* k_cache, const void* v_cache, int32_t kv_format, int32_t num_pages,
                     const float* k_scale, const float* v_scale, const int32_t* block_table, int64_t bt_stride,
                     int32_t bt_cols, void* k_out, void* v_out, int32_t out_format, int64_t so_kb, int64_t so_kh,
                     int64_t so_ks, int64_t so_vb, int64_t so_vh, int64_t so_vs, int32_t batch, int32_t kv_heads,
                     int32_t keys, int32_t head_dim, int32_t page_size, void* stream);

/* The dense view of the paged KIVI cache, as eco_paged_gather: keys below keys_quantized[b] and values below
 * values_quantized[b] dequantized as the reference's dequantize (bf16(code * scale + zero), attention/kivi.py:
 * 56-76), the other tokens from the rings. Replaces KIVIPacked's materialize (attention/packed.py:66-78). */
int eco_kivi_gather(const void* blocks, int32_t num_pages, const void* k_ring, const void* v_ring, int32_t ring,
                    const int32_t* keys_quantized, const int32_t* values_quantized, const int32_t* block_table,
                    int64_t bt_stride, int32_t bt_cols, void* k_out, void* v_out, int32_t out_format, int64_t so_kb,
                    int64_t so_kh, int64_t so_ks, int64_t so_vb, int64_t so_vh, int64_t so_vs, int32_t batch,
                    int32_t kv_heads, int32_t keys, int32_t head_dim, int32_t bits, int32_t group, void* stream);

/* Workspace bytes eco_decode needs for this shape (0 for an unsupported one). The workspace starts with a counter per
 * block of 16 query rows, int32 per batch row, KV head and block of 16 of the (q_heads / kv_heads) * queries rows,
 * padded to 256 bytes, which must be zero when a call starts; every call leaves them zero and may write anything after
 * them (the counter rule of eco_paged_decode's workspace). One workspace serves one stream at a time. */
size_t eco_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys,
                                 int32_t head_dim, int32_t value_dim);

/* Decode attention over dense K/V buffers: out[b, qi, h, :] (element strides so_*, the query's format) for query
 * q[b, h, qi, :] (format q_format = bf16, fp16 or fp32; element strides sq_*), over k [b, kvh, t, :] and v
 * [b, kvh, t, :] (t < keys; element strides sk_*, sv_*; format kv_format = the query's, or fp8 e4m3 / e5m2 with
 * optional per-head scales k_scale / v_scale [Hkv]), query head h reading KV head h / (q_heads / kv_heads). The
 * optional boolean mask (one byte per element, element mask[b * sm_b + h * sm_h + qi * sm_q + t * sm_s], stride 0
 * for a broadcast dimension) hides the keys where it is 0; without it every key is visible. Scores are
 * q . k * scale, with an optional soft cap (softcap > 0) and sinks [Hq] in the denominator; a query that sees no key
 * gives 0. Channel strides are 1; head_dim and value_dim are multiples of 8 (of 16 for fp8), at most 512 (at most 256
 * for fp32 K/V; heads wider than 256 run as value slices of 256 channels, attention/decode.py:216-232); pointers
 * and K/V/query strides are 16-byte aligned. Replaces decode_attention (attention/decode.py:252-324; kernels
 * attention/_decode_kernels.py:78-226): split-K over the keys, the splits merged by the last of their waves. */
int eco_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
               const void* v, int32_t kv_format, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b, int64_t sv_h,
               int64_t sv_s, const float* k_scale, const float* v_scale, const uint8_t* mask, int64_t sm_b,
               int64_t sm_h, int64_t sm_q, int64_t sm_s, const float* sinks, void* out, int64_t so_b, int64_t so_q,
               int64_t so_h, int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys,
               int32_t head_dim, int32_t value_dim, float scale, float softcap, void* workspace,
               size_t workspace_bytes, void* stream);

/* Quest page bounds: kmin / kmax (bf16 [B, Hkv, P, D], element strides sb_b, sb_h, sb_p, channel stride 1) of the
 * Quest pages [first, last) of every row (quest_page_size tokens each, a power of two >= 16), the channel-wise
 * smallest and largest stored key read through the block table (fp8 decoded exactly; per-head scales not applied:
 * they scale every score of a (row, KV head) alike). A Quest page with a cache page outside the table or the cache
 * is left untouched. Replaces page_bounds (attention/quest.py:54-65) as QuestCache._layer_bounds calls it
 * (techniques/quest/technique.py:229-259). */
int eco_quest_page_bounds(const void* k_cache, int32_t kv_format, int32_t num_pages, const int32_t* block_table,
                          int64_t bt_stride, int32_t bt_cols, int32_t first, int32_t last, int32_t quest_page_size,
                          void* kmin, void* kmax, int64_t sb_b, int64_t sb_h, int64_t sb_p, int32_t batch,
                          int32_t kv_heads, int32_t head_dim, int32_t page_size, void* stream);

/* Quest page bounds kept on append, every range on the device: for each row b and KV head h, the bounds of the Quest
 * pages [valid[b * Hkv + h], min(committed[b] / quest_page_size, page_cap)) are computed as eco_quest_page_bounds
 * does, then valid advances to that end and done[b] (optional) becomes the row's committed Quest pages. The launch
 * shape depends on the arguments only, so a decode step can be captured in a graph; valid starts at zero.
 * Replaces QuestCache.pass_begin / _layer_bounds with its host done list (techniques/quest/technique.py:165-172,
 * 229-259), which keeps the reference's Quest out of graphs (technique.py:311). */
int eco_quest_refresh_bounds(const void* k_cache, int32_t kv_format, int32_t num_pages, const int32_t* block_table,
                             int64_t bt_stride, int32_t bt_cols, const int32_t* committed, int32_t* valid,
                             int32_t* done, int32_t quest_page_size, void* kmin, void* kmax, int64_t sb_b,
                             int64_t sb_h, int64_t sb_p, int32_t page_cap, int32_t batch, int32_t kv_heads,
                             int32_t head_dim, int32_t page_size, void* stream);

/* Workspace bytes of eco_quest_select (the page scores, fp32 [B, Hkv, max_done]). */
size_t eco_quest_select_workspace_size(int32_t batch, int32_t kv_heads, int32_t max_done);

/* Quest page selection: out[b, kvh, 0..pages) (int32, contiguous) = the pages of row b with the largest scores
 * sum_d qsum_d (lo + hi) / 2 + qabs_d (hi - lo) / 2 among its committed pages [0, done[b]) (pages >= max_done never),
 * min(pages, max_done) of them in increasing order, then -1; ties go to the lower page. qsum / qabs are the fp32
 * sums of q / |q| (q [B, Q, Hq, D] in q_format = bf16, fp16 or fp32, element strides sq_*, channel stride 1) over
 * the KV head's query rows; lo / hi are the page bounds (bounds_format = bf16, fp16 or fp32, 16-byte aligned,
 * strides multiples of 8 elements), all widened to fp32 exactly. Replaces select_pages (attention/quest.py:73-108).
 * first_page nonzero always selects a row's page 0 (it scores +inf), the "first and last pages" variant of Quest;
 * the reference has no such rule, so 0 gives its selection. */
int eco_quest_select(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* kmin,
                     const void* kmax, int32_t bounds_format, int64_t sb_b, int64_t sb_h, int64_t sb_p,
                     const int32_t* done, int32_t max_done, int32_t pages, int32_t first_page, int32_t* out,
                     int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Quest page bounds over a dense key buffer (the reference's own cache layout): kmin / kmax [b, h, p, :] (element
 * strides sb_*, channel stride 1; page p written at p * sb_p) of pages [first, last) of page_size slots (a power of
 * two >= 16; last * page_size <= slots), the channel-wise smallest and largest key of keys [b, h, s, :] (element
 * strides sk_*, channel stride 1; format kv_format = bf16, fp16, fp32 or fp8) with NaN propagated as torch's amin /
 * amax do. bounds_format must be bounds_dtype's: bf16 for bf16 and fp8 keys (exact), else the keys' format.
 * Replaces page_bounds and bounds_dtype (attention/quest.py:54-70) as QuestCache._layer_bounds calls them
 * (techniques/quest/technique.py:229-259). */
int eco_quest_dense_bounds(const void* keys, int32_t kv_format, int64_t sk_b, int64_t sk_h, int64_t sk_s,
                           int32_t slots, int32_t first, int32_t last, int32_t page_size, void* kmin, void* kmax,
                           int32_t bounds_format, int64_t sb_b, int64_t sb_h, int64_t sb_p, int32_t batch,
                           int32_t kv_heads, int32_t head_dim, void* stream);

/* Workspace bytes of eco_quest_decode: eco_decode_workspace_size over the virtual key axis
 * pages * page_size + keys - min_done * page_size (at least 1), with eco_decode's counter rule. */
size_t eco_quest_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                                       int32_t keys, int32_t pages, int32_t page_size, int32_t min_done,
                                       int32_t head_dim, int32_t value_dim);

/* Quest decode attention over dense K/V buffers: eco_decode over the virtual key axis of (row b, KV head h) made of
 * the selected pages index[b, h, 0 .. pages) (element strides si_b, si_h; increasing, then -1; page i covers slots
 * i * page_size .. + page_size) in slot order, then the dense tail, slots done[b] * page_size .. keys. The optional
 * mask is over slots (a selected page's key carries its slot's mask column). min_done = min(done) on the host sizes
 * the split plan; the launch shape is a function of the shapes and min_done. Everything else as eco_decode (query
 * bf16 / fp16 / fp32, K/V in its format or fp8 with per-head scales, soft cap, sinks, a query that sees no key gives
 * 0). Entries outside the buffer's whole pages are clamped (wrong results, no access outside a buffer). Replaces
 * quest_decode_attention (attention/quest.py:239-344; kernel attention/_quest_kernels.py:13-97). */
int eco_quest_decode(const void* q, int32_t q_format, int64_t sq_b, int64_t sq_h, int64_t sq_q, const void* k,
                     const void* v, int32_t kv_format, int64_t sk_b, int64_t sk_h, int64_t sk_s, int64_t sv_b,
                     int64_t sv_h, int64_t sv_s, const float* k_scale, const float* v_scale, const int32_t* index,
                     int64_t si_b, int64_t si_h, int32_t pages, const int32_t* done, int32_t page_size,
                     int32_t min_done, const uint8_t* mask, int64_t sm_b, int64_t sm_h, int64_t sm_q, int64_t sm_s,
                     const float* sinks, void* out, int64_t so_b, int64_t so_q, int64_t so_h, int32_t batch,
                     int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t keys, int32_t head_dim,
                     int32_t value_dim, float scale, float softcap, void* workspace, size_t workspace_bytes,
                     void* stream);

/* ---- KIVI (2- and 4-bit KV codes) --------------------------------------------------------------------------
 * Paged KIVI cache, per layer: blocks [num_pages, Hkv, eco_kivi_block_bytes] (one block per 32-token page and KV
 * head: key codes, value codes, key scales and zero points per channel of the page's 32-token key group, value scales
 * and zero points per token and 32-channel group; fp16), and the full-precision residual of every row in two bf16
 * rings of W slots (token t at slot t % W): keys [B, Hkv, W, D], values [B, Hkv, D, W]. Keys below
 * keys_quantized[b] and values below values_quantized[b] (int32 [B] on the device) are read from the pages, the
 * others from the rings. Row b's token t lives in page block_table[b * bt_stride + t / 32]. */

/* Bytes of one (page, KV head) block (0 for an unsupported shape: head dim 64 or 128, 2 or 4 bits, group 32). */
size_t eco_kivi_block_bytes(int32_t head_dim, int32_t bits, int32_t group);

/* The reference's KIVI schedule (techniques/kv_quant/kivi.py:230-243) on the device: with committed[b] tokens, keys
 * below (c / residual) * residual and values below max(0, c - residual) are quantized. Writes ranges int32 [4, B]
 * (keys from, keys to, values from, values to: what to quantize now) and advances keys_quantized / values_quantized. */
int eco_kivi_schedule(const int32_t* committed, int32_t residual, int32_t group, int32_t* keys_quantized,
                      int32_t* values_quantized, int32_t* ranges, int32_t batch, void* stream);

/* KIVI quantize-and-append: quantizes tokens [from[b], to[b]) of every row into its pages, keys (kind 0, per channel
 * over 32-token groups; from and to multiples of 32) or values (kind 1, per token over 32-channel groups). The source
 * element (b, h, t, d) is at src + b * ss_b + h * ss_h + slot * ss_t + d * ss_d (elements of src_format), slot =
 * t - src_start, or t % src_ring with a ring. max_tokens bounds to - from over the rows (it sizes the launch). A scale
 * or zero point beyond fp16 sets *overflow (optional). Replaces quantize / pack_codes as FusedKIVICache._quantize_block
 * and the paged _quantize_kernel call them (techniques/kv_quant/kivi.py:121-140, attention/kivi.py:38-45,
 * techniques/kv_kivi_fused/fused.py:152-175, backends/vllm/kivi/kernels.py:94-207). */
int eco_kivi_quantize(int32_t kind, const void* src, int32_t src_format, int64_t ss_b, int64_t ss_h, int64_t ss_t,
                      int64_t ss_d, int32_t src_start, int32_t src_ring, const int32_t* from, const int32_t* to,
                      void* blocks, int32_t num_pages, const int32_t* block_table, int64_t bt_stride,
                      int32_t bt_cols, int32_t batch, int32_t kv_heads, int32_t head_dim, int32_t bits,
                      int32_t group, int32_t max_tokens, uint32_t* overflow, void* stream);

/* KIVI's simulated storage: quantizes slots [start, stop) of every row of a dense buffer [B, H, slots, D] (element
 * strides sb, sh, ss, channel stride 1; bf16, fp16 or fp32) in place, keys (keys = 1: per channel over groups of
 * `group` tokens, stop - start a multiple of group) or values (keys = 0: per token over groups of `group` channels,
 * group dividing D), each element replaced by code * scale + low in fp32 rounded to the buffer's dtype; bits 2, 4 or
 * 8, any group. Replaces KIVICache._quantize_block / _quantize with quantize and fake_quantize
 * (techniques/kv_quant/kivi.py:110-140, 257-275). */
int eco_kivi_fake_quantize(void* buffer, int32_t format, int64_t sb, int64_t sh, int64_t ss, int32_t batch,
                           int32_t heads, int32_t slots, int32_t head_dim, int32_t start, int32_t stop, int32_t bits,
                           int32_t group, int32_t keys, void* stream);

/* KIVI's packed record (the reference's KIVIPacked layout, attention/kivi.py:80-132) written from a dense buffer or a
 * ring: for every row b, slots [from[b], to[b]) (int32 [B] on the device, clamped to [0, slots); keys: multiples of
 * group) of src [B, H, *, D] (element strides ss_*, channel stride 1; bf16, fp16 or fp32; slot s at s % src_ring when
 * src_ring > 0) are quantized as the reference's quantize (techniques/kv_quant/kivi.py:121-140): keys (kind 0) per
 * channel over groups of `group` tokens, values (kind 1) per token over groups of `group` channels (group dividing
 * D). Codes go to codes [B, H, slots, D * bits / 8] (byte strides sc_*; packed as pack_codes, attention/kivi.py:
 * 38-45), fp16 scales and zero points to scale / zero (element strides sz_*; keys [B, H, ceil(slots / group), D] at
 * row s / group, values [B, H, slots, D / group]). write_back (not with a ring): every source element is replaced by
 * code * scale + low in fp32 rounded to its format, the dense values of the reference's fused cache. max_tokens bounds
 * to - from over the rows (it sizes the launch; keys: a multiple of group). *overflow (optional) is set to 1 when a
 * scale or zero point lies beyond fp16 (its fp16 copy is then not the value the codes were made with). Replaces
 * FusedKIVICache._quantize_block and PackedKIVICache._pack_block (techniques/kv_kivi_fused/fused.py:152-175,
 * techniques/kv_quant/packed.py:213-230). */
int eco_kivi_pack_quantize(int32_t kind, void* src, int32_t format, int64_t ss_b, int64_t ss_h, int64_t ss_s,
                           int32_t src_ring, int32_t write_back, void* codes, int64_t sc_b, int64_t sc_h, int64_t sc_s,
                           void* scale, void* zero, int64_t sz_b, int64_t sz_h, int64_t sz_s, const int32_t* from,
                           const int32_t* to, int32_t batch, int32_t heads, int32_t slots, int32_t head_dim,
                           int32_t bits, int32_t group, int32_t max_tokens, uint32_t* overflow, void* stream);

/* The dense view of a KIVI packed record's keys (kind 0) or values (kind 1): out [B, H, slots, D] (element strides
 * so_*, format bf16 / fp16 / fp32) holds code * scale + zero in fp32 rounded to the format where slot s <
 * quantized[b] (codes, scale, zero as eco_kivi_pack_quantize lays them out), and the full-precision entry of `ring`
 * [B, H, *, D] (element strides sr_*, the output's format) at slot s % ring_slots (slot s when ring_slots is 0)
 * elsewhere. quantized[b] must not exceed the slots the codes hold. Replaces PackedKIVICache._dense
 * (techniques/kv_quant/packed.py:300-320), the dense copy read by attention paths that do not read codes. */
int eco_kivi_packed_gather(int32_t kind, const uint8_t* codes, int64_t sc_b, int64_t sc_h, int64_t sc_s,
                           const void* scale, const void* zero, int64_t sz_b, int64_t sz_h, int64_t sz_s,
                           const int32_t* quantized, const void* ring, int64_t sr_b, int64_t sr_h, int64_t sr_s,
                           int32_t ring_slots, void* out, int32_t format, int64_t so_b, int64_t so_h, int64_t so_s,
                           int32_t batch, int32_t heads, int32_t slots, int32_t head_dim, int32_t bits, int32_t group,
                           void* stream);

/* KIVI's cell on vLLM's paged cache (backends/vllm/kivi/layout.py:133-213): for a head size (a power of two, 16 to
 * 256) of a cache dtype of element_size bytes, bits 2 / 4 / 8 and a power-of-two group of at most 128, writes
 * offsets[10] = {value group, key aux slots, off_v, off_vs, off_vz, off_ka, off_kc, off_vc, off_flag, cell bytes}. */
int eco_kivi_cells_layout(int32_t head_dim, int32_t element_size, int32_t bits, int32_t group, int32_t* offsets);

/* The reference's quantize_committed (backends/vllm/kivi/kernels.py:94-207) on the cells of one layer's cache
 * [pages, kv_heads, page_size] (cell byte strides sb, sh, sn, dense entries of format bf16 / fp16 / fp32): for every
 * request not prefilling with a non-empty query (query_start_loc [requests + 1]) and c = seq_lens[b] - its query
 * length > 0, keys in whole groups below (c / residual) * residual and values below c - residual, newest first, until
 * a cell already quantized; cells laid out as write_cells does (layout.py:222-256): dense entries replaced by the
 * dequantized values, codes, fp16 scales and zero points, flags 1 (2: a scale or zero point beyond fp16). plan: device
 * scratch of 4 int32 per (request, KV head), any contents (the walk's stopping points, found over the flags before
 * any cell changes; the groups and tokens are then quantized by many workgroups per request and head). */
int eco_kivi_cells_quantize(void* cache, int32_t format, int64_t sb, int64_t sh, int64_t sn, int32_t num_pages,
                            int32_t page_size, int32_t kv_heads, const int32_t* block_table, int64_t bt_stride,
                            int32_t bt_cols, const int32_t* query_start_loc, const int32_t* seq_lens,
                            const int32_t* prefilling, int32_t requests, int32_t head_dim, int32_t bits,
                            int32_t group, int32_t residual, int32_t* plan, void* stream);

/* The reference's paged_kivi_attention (backends/vllm/kivi/kernels.py:216-415) over the cells of one layer's cache
 * [pages, kv_heads, page_size] (byte strides sb, sh, sn; entries and queries of format bf16 / fp16 / fp32): vLLM's
 * varlen queries q [tokens, q_heads, D] (element strides sq_t, sq_h; request b's queries are tokens
 * query_start_loc[b] .. query_start_loc[b + 1] - 1, at most max_query_len), each attending causally over its
 * request's seq_lens[b] keys (query i of a request of n queries sees keys < seq_len - n + i + 1); out
 * [tokens, q_heads, D] (strides so_t, so_h); keys = the longest seq_len (at least every seq_lens[b]); optional sinks
 * [q_heads] and soft cap. As the reference's kernel (kernels.py:274-296), a key or value whose cell flag is 1 is read
 * through its codes, value scales and zero points and its key group's scales and zero points, and its dense entry is
 * ignored, for bf16 cells of 128 channels, key groups of 32, 2- or 4-bit codes and page_size a multiple of 32; any
 * other flag, any other cell shape, and every cell when the environment sets ECO_CELLS_DENSE=1, is read from its
 * dense entry (which eco_kivi_cells_quantize leaves holding the dequantized value). block_table has a row per
 * request. Workspace:
 * eco_kivi_cells_attention_workspace_size bytes, with eco_decode's counter rule (batch = requests, queries =
 * max_query_len). */
size_t eco_kivi_cells_attention_workspace_size(int32_t requests, int32_t max_query_len, int32_t q_heads,
                                               int32_t kv_heads, int32_t keys, int32_t head_dim);
int eco_kivi_cells_attention(const void* q, int64_t sq_t, int64_t sq_h, const void* cache, int32_t format, int64_t sb,
                             int64_t sh, int64_t sn, int32_t num_pages, int32_t page_size, int32_t kv_heads,
                             const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                             const int32_t* query_start_loc, const int32_t* seq_lens, int32_t requests,
                             int32_t max_query_len, int32_t keys, int32_t head_dim, int32_t bits, int32_t group,
                             const float* sinks, void* out, int64_t so_t, int64_t so_h, int32_t q_heads, float scale,
                             float softcap, void* workspace, size_t workspace_bytes, void* stream);

/* clear_flags (kernels.py:58-78): the cells of slots[tokens] (page * page_size + position; negative: padding) of
 * every KV head marked full precision (both flags 0), after vLLM's cache write filled them. */
int eco_kivi_cells_clear_flags(void* cache, int32_t format, int64_t sb, int64_t sh, int64_t sn, int32_t num_pages,
                               int32_t page_size, int32_t kv_heads, const int32_t* slots, int32_t tokens,
                               int32_t head_dim, int32_t bits, int32_t group, void* stream);

/* Writes new tokens k_new / v_new [T, Hkv, D] (element strides, channel stride 1) into the rings at slot
 * positions[t] % ring of row rows[t] (negative positions skip), rounded to bf16 (the reference's ring writes,
 * kv_quant/packed.py:258-277). */
int eco_kivi_ring_write(const void* k_new, const void* v_new, int32_t in_format, int64_t sk_t, int64_t sk_h,
                        int64_t sv_t, int64_t sv_h, const int32_t* rows, const int32_t* positions, int32_t tokens,
                        void* k_ring, void* v_ring, int32_t batch, int32_t kv_heads, int32_t head_dim, int32_t ring,
                        void* stream);

/* Workspace bytes eco_kivi_decode needs; the same layout and counter rule as eco_paged_decode's workspace. */
size_t eco_kivi_decode_workspace_size(int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads,
                                      int32_t head_dim, int32_t max_seq_len, int32_t bits);

/* Decode attention over the paged KIVI cache and the rings: as eco_paged_decode (query [B, Q, Hq, D] bf16, out
 * [B, Q, Hq, D] bf16, causal over the last Q of seq_lens[b] tokens, soft cap, sinks), with keys below
 * keys_quantized[b] (whole 32-token key groups, as eco_kivi_schedule counts them) and values below
 * values_quantized[b] read as codes; more than 64 query rows per KV head in query chunks as eco_paged_decode. Replaces
 * kivi_decode_attention (attention/kivi.py:199-309) and paged_kivi_attention (backends/vllm/kivi/kernels.py:354-415). */
int eco_kivi_decode(const void* q, int64_t sq_b, int64_t sq_q, int64_t sq_h, const void* blocks, int32_t num_pages,
                    const void* k_ring, const void* v_ring, int32_t ring, const int32_t* keys_quantized,
                    const int32_t* values_quantized, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                    const int32_t* seq_lens, const float* sinks, void* out, int64_t so_b, int64_t so_q, int64_t so_h,
                    int32_t batch, int32_t queries, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                    int32_t bits, int32_t group, int32_t max_seq_len, float scale, float softcap,
                    const uint32_t* mask_bits, int64_t mk_b, int64_t mk_h, int64_t mk_q, int32_t mask_words,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Decode attention over a KIVI packed record of dense-layout codes (the reference's KIVIPacked, attention/kivi.py:
 * 80-132): eco_decode's call (query q_format = bf16, fp16 or fp32 with k / v in the same format, mask, soft cap,
 * sinks, workspace of eco_decode_workspace_size) where, for row b, keys t < keys_quantized[b] and values t <
 * values_quantized[b] (int32 [B] on the device, clamped to [0, keys]) are code * scale + zero computed in fp32 and
 * rounded to the query's format, from
 *   key_codes   uint8 [B, Hkv, keys, D * bits / 8] (byte strides skc_*; channel d in byte d * bits / 8 at bit
 *               (d % (8 / bits)) * bits, as pack_codes packs them, attention/kivi.py:38-45),
 *   key_scale / key_zero   fp16 [B, Hkv, ceil(keys / key_group), D] (element strides sks_*, shared),
 *   value_codes uint8 [B, Hkv, keys, Dv * bits / 8] (byte strides svc_*),
 *   value_scale / value_zero   fp16 [B, Hkv, keys, Dv / value_group] (element strides svs_*, shared),
 * bits 2, 4 or 8, any key group, a value group dividing Dv; every other key and value is read from k / v at slot t,
 * or, with ring > 0, from the rings k / v at slot t % ring (the reference's key_ring / value_ring). The result is
 * bit-identical to eco_decode over buffers holding the dequantized values. Alignment: codes and their strides to the
 * bytes of 16 / element_size codes, key scales to 16 / (8 for fp32) bytes with strides in multiples of 8 (4)
 * elements. Replaces kivi_decode_attention (attention/kivi.py:199-309; kernel attention/_kivi_kernels.py:14-326). */
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
                           float softcap, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ECONOMIZE_AMD_H */
