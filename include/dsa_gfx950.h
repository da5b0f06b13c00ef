/*
 * dsa_gfx950.h — C ABI of the MI355X (gfx950) DeepSeek-Sparse-Attention decode path:
 * lightning indexer -> exact per-row top-k -> sparse MLA attention over a paged FP8 KV cache.
 *
 * Every pointer is a device pointer unless stated otherwise; every entry point enqueues work on `stream`
 * (a hipStream_t passed as void*) and returns without synchronising (dsa_layer_status excepted). Return value:
 * DSA_OK (0) or a negative DSA_E* code; dsa_strerror() names it. No entry point allocates device memory: scratch
 * space is a caller-owned workspace sized by dsa_workspace_bytes(). A workspace must be zero-filled before its
 * first use (dsa_workspace_clear, or any zero fill) and written by nothing but these calls afterwards. A decode or
 * top-k workspace starts with 8 KiB of barrier and status words at the same offset for every batch size (a barrier
 * counter only grows, by 256 per launch that uses it, so it always holds a multiple of 256 between calls, zero
 * included; the status words count across calls, see dsa_layer_status), then the top-k histograms [B, 4096] int32:
 * with the barrier words, the zero region of a call of B rows, which the call leaves as it found it (histograms zero,
 * counters multiples of 256); the rest is per-call scratch. The library records on the host
 * how much of each workspace's start is zero and zero-fills the difference (a fill kernel on the call's stream)
 * before a call whose zero region reaches further than the last call's, or before the first call it sees on a
 * workspace: so one workspace serves any number of calls, of any batch sizes it is large enough for, and graph
 * replays. Calls that share a workspace must not overlap.
 * Kernels never raise; every shape and argument check happens on the host before launch, so a call that returns
 * DSA_EINVAL, DSA_EUNSUPPORTED or DSA_EWORKSPACE has written nothing. After a call that returns DSA_ELAUNCH the next
 * call on its workspace zero-fills the whole zero region first.
 *
 * Cache layout (the paged FP8 cache of trnrt/models/decoder.py:459-490 and trnrt/engine/model_runner.py:54-70,
 * extended with per-token scales):
 *   - a cache holds num_pages * page_size token slots; page 0 is the null page (trnrt/engine/kv_pool.py:1-15);
 *   - token t of sequence b lives in slot page_table[b * max_pages + t / page_size] * page_size + t % page_size
 *     (trnrt/models/decoder.py:658-667);
 *   - indexer keys: uint8 OCP e4m3fn [slots, D] + fp32 per-token scale [slots] (key = k_fp8 * k_scale);
 *   - latent KV: uint8 OCP e4m3fn [slots, Dqk] (Dqk = 512 latent + 64 rope) + fp32 per-token scale [slots].
 * Page ids outside [0, num_pages) read the null page instead of faulting.
 */
#ifndef DSA_GFX950_H
#define DSA_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_ABI_VERSION 10

#define DSA_OK 0
#define DSA_EINVAL (-1)      /* a null pointer or a size out of range */
#define DSA_EUNSUPPORTED (-2) /* a shape these kernels do not implement */
#define DSA_EWORKSPACE (-3)  /* workspace smaller than dsa_workspace_bytes() */
#define DSA_ELAUNCH (-4)     /* the HIP runtime refused a launch */
#define DSA_ESCRATCH (-5)    /* more scratch than dsa_decode_layer_noalloc holds */

/* Workspace kinds for dsa_workspace_bytes(). */
#define DSA_WS_TOPK 1
#define DSA_WS_ATTENTION 2
#define DSA_WS_LAYER 3

int dsa_abi_version(void);
const char* dsa_strerror(int status);

/*
 * Decode indexer scores (replaces trnrt/kernels/dsa_index.py:243-268 `scores`, arithmetic of
 * dsa_index.py:44-50 `emulate` and trnrt/models/dsa_long.py:74-84 `scores`):
 *   scores[b, t] = k_scale[slot(b,t)] * sum_h w[b, h] * relu(q[b, h, :] . k_fp8[slot(b,t), :]) + cand[b, t]
 * for t < ctx_len[b]; NEG_INF (-1e30) for ctx_len[b] <= t < score_stride.
 *   q        bf16 [B, Hi, D]          (D must be 128; Hi <= 64)
 *   w        fp32 [B, Hi]             head weights with D^-0.5 already folded in (trnrt/models/mla.py:629)
 *   k_fp8    uint8 [num_pages * page_size, D], k_scale fp32 [num_pages * page_size]
 *   page_table int32 [B, max_pages],  ctx_len int32 [B] (values clamped to max_pages * page_size)
 *   cand     fp32 [B, score_stride] additive (0 / NEG_INF) or NULL
 *   scores   fp32 [B, score_stride];  page_size a multiple of 32; score_stride <= max_pages * page_size
 */
int dsa_indexer_decode(const void* q_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                       const int32_t* page_table, const int32_t* ctx_len, const float* cand, float* scores, int B,
                       int Hi, int D, int max_pages, int page_size, int num_pages, int score_stride, void* stream);

/*
 * Decode indexer scores over a bf16 key cache with no per-key scale: GLM's pooled indexer over its pool-key cache
 * (replaces trnrt/kernels/dsa_index.py:243-268 `scores` as called at trnrt/models/mla.py:628-629, one key per pool):
 *   scores[b, p] = sum_h w[b, h] * relu(q[b, h, :] . k_bf16[slot(b, p), :]) (+ cand[b, p]),  NEG_INF at p >= ctx_len[b]
 *   slot(b, p) = page_table[b, p / page_size] * page_size + p % page_size (page_size keys per page, any >= 1; 16 pools
 *   of kpool 4 in a 64-token page); k_bf16 [num_pages * page_size, D]; other arguments as dsa_indexer_decode.
 */
int dsa_indexer_decode_bf16(const void* q_bf16, const float* w, const void* k_bf16, const int32_t* page_table,
                            const int32_t* ctx_len, const float* cand, float* scores, int B, int Hi, int D,
                            int max_pages, int page_size, int num_pages, int score_stride, void* stream);

/*
 * Dense (prefill-chunk) indexer scores of N queries over one context's keys (replaces the score stage of
 * trnrt/kernels/dsa_long_select.py:500-530 `select`, arithmetic of dsa_long_select.py:119-133 `emulate_scores`
 * and trnrt/models/dsa_long.py:74-84 `scores` with a 2-D key tensor):
 *   scores[n, p] = scale * k_scale[p] * sum_h w[n, h] * relu(q[n, h, :] . k_fp8[p, :])   for p < npool[n]
 *   scores[n, p] = NEG_INF                                                               for npool[n] <= p < score_stride
 *   q bf16 [N, Hi, D] (D must be 128; Hi <= 64), w fp32 [N, Hi], k uint8 e4m3 [P, D] + k_scale fp32 [P], or
 *   k bf16 [P, D] with k_scale null (GLM's pool keys, trnrt/models/mla.py:491-503; then Hi <= 32), npool int32 [N]
 *   (each query's candidate count, clamped to [0, P]), scores fp32 [N, score_stride], P <= score_stride.
 */
int dsa_indexer_prefill(const void* q_bf16, const float* w, const void* k, const float* k_scale,
                        const int32_t* npool, float* scores, int N, int Hi, int D, int P, int score_stride,
                        float scale, void* stream);

/*
 * The same scores with FP8 e4m3 queries and a per-(query, head) fp32 scale (the indexer's FP8 query form; the
 * reference's arithmetic on the dequantised queries q = q_fp8 * q_scale, trnrt/kernels/dsa_long_select.py:119-133):
 *   scores[n, p] = scale * k_scale[p] * sum_h w[n, h] q_scale[n, h] * relu(q_fp8[n, h, :] . k_fp8[p, :])
 *   q_fp8 uint8 [N, Hi, D] (e4m3fn bits; D must be 128; Hi <= 64), q_scale fp32 [N, Hi] (positive); the rest as
 *   dsa_indexer_prefill.
 */
int dsa_indexer_prefill_fp8(const uint8_t* q_fp8, const float* q_scale, const float* w, const uint8_t* k_fp8,
                            const float* k_scale, const int32_t* npool, float* scores, int N, int Hi, int D, int P,
                            int score_stride, float scale, void* stream);

/*
 * Exact top-k per row (replaces trnrt/models/dsa_long.py:140-186 `select_device` and the selection of
 * trnrt/kernels/dsa_topk.py:495-514 `select`; rule of trnrt/models/dsa_select.py:10-38): per row b over positions
 * t < min(len[b], score_stride), the `keep` largest scores, ties at the keep-th value to the lowest positions;
 * only scores > VISIBLE (-5e29) are selectable when vis_only != 0; -0.0 == +0.0; NaN is not allowed.
 * Output: idx int32 [B, keep] the selected positions ascending, 0 past cnt; cnt int32 [B] = min(keep, #selectable).
 *   len      int32 [B] or NULL (NULL: score_stride for every row)
 *   max_len  an upper bound of the row lengths (sizes the launch; <= score_stride)
 *   workspace  dsa_workspace_bytes(DSA_WS_TOPK, B, 0, keep, max_len, 0) bytes, zero-filled before first use
 */
int dsa_topk(const float* scores, const int32_t* len, int32_t* idx, int32_t* cnt, void* workspace,
             size_t workspace_bytes, int B, int score_stride, int max_len, int keep, int vis_only, void* stream);

/* Zero-fills workspace (16-byte aligned, bytes a multiple of 16) with a kernel on `stream` (no memset node, so a
 * captured graph may contain it). */
int dsa_workspace_clear(void* workspace, size_t workspace_bytes, void* stream);

/* 1 if dsa_topk implements rows of up to max_len scores at this keep (and vis_only), else 0. */
int dsa_topk_supported(int max_len, int keep, int vis_only);

/*
 * Additive selection mask (the output form of trnrt/kernels/dsa_topk.py:495-514 `select`, with its pooled kp and
 * tail forms, dsa_topk.py:89-93): score p of row b (P scores per row) is taken when it is one of idx[b, 0 ..
 * cnt[b]), or, with tail, when it is not a candidate (scores[b, p] <= VISIBLE: the reference's `sel | ~vis`);
 * mask[b, p * kp + t] = taken ? 0 : NEG_INF for t < kp. scores (fp32 [B, P]) is read only with tail.
 * idx and cnt NULL: the form of keep >= P (dsa_topk.py:510-511, no selection run): every score that scores marks
 * visible (scores[b, p] > VISIBLE) is taken, or every score when scores is NULL; tail as above.
 */
int dsa_topk_mask(const int32_t* idx, const int32_t* cnt, const float* scores, float* mask, int B, int keep, int P,
                  int kp, int tail, void* stream);

/*
 * Sparse MLA decode attention over the selected tokens (replaces trnrt/kernels/dsa_decode.py:26-43 `attend`,
 * trnrt/kernels/dsa_slots.py:48-65 `emulate` with lse, trnrt/models/dsa_long.py:189-223 `slots` + `attend`; split
 * combine of trnrt/models/mla.py:853-856):
 *   K[k] = kv_fp8[slot_k, :Dqk] * kv_scale[slot_k] (key, Dqk = 576: 512 latent + 64 rope, or 512: GLM's NoPE latent;
 *   rows of Dqk bytes), V[k] = K[k][:Dv] (Dv = 512); kv_scale NULL: every scale 1 (the reference's unscaled FP8
 *   cache, trnrt/models/decoder.py:481-486; so in every entry point below that takes a kv_scale)
 *   s[h, k] = scale * q[b, h, :] . K[k] + bias_k,  p = softmax_k(s),  out[b, h, :] = sum_k p[h, k] V[k]
 *   lse[b, h] = max_k s + log sum_k exp(s - max)
 * Two ways to name the slots (exactly one must be given):
 *   token form: idx int32 [B, keep] token positions + cnt int32 [B] + page_table int32 [B, max_pages];
 *               bias_k = 0 for k < cnt[b], NEG_INF otherwise (cnt 0 attends position 0 with lse NEG_INF);
 *   row form:   rows int32 [B, keep] cache slots + bias fp32 [B, keep] additive (0 / NEG_INF);
 *               page_table and cnt are ignored (may be NULL).
 *   q bf16 [B, H, Dqk] (H a multiple of 16), out bf16 [B, H, Dv] or NULL, out_f32 fp32 [B, H, Dv] or NULL,
 *   lse fp32 [B, H] or NULL; splits >= 1 (0: chosen for the GPU) partitions the keep slots across workgroups.
 */
int dsa_sparse_mla_decode(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* idx,
                          const int32_t* cnt, const int32_t* page_table, const int32_t* rows, const float* bias,
                          void* out_bf16, float* out_f32, float* lse, void* workspace, size_t workspace_bytes, int B,
                          int H, int Dqk, int Dv, int keep, int max_pages, int page_size, int num_pages, float scale,
                          int splits, void* stream);

/*
 * Slot attention over the first n rows of N, n read on the device (replaces trnrt/kernels/dsa_slots_n.py:154-203
 * `attend`, whose n is a one-element int tensor and whose rows past n stay unwritten on the device): the row form of
 * dsa_sparse_mla_decode (rows int32 [N, keep] cache slots of kv_fp8 [num_slots, Dqk], bias fp32 [N, keep]) over rows
 * r < *n_live only; out / out_f32 / lse rows at or past it are not written (no work is done for them). n_live: int32
 * [1] on the device (values past N act as N). Workspace as dsa_sparse_mla_decode's at (N, H, keep, splits).
 */
int dsa_sparse_mla_slots_n(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* rows,
                           const float* bias, const int32_t* n_live, void* out_bf16, float* out_f32, float* lse,
                           void* workspace, size_t workspace_bytes, int N, int H, int Dqk, int keep,
                           long long num_slots, float scale, int splits, void* stream);

/*
 * Mask compaction (trnrt/models/dsa_long.py:140-166 `compact`): row n of sel fp32 [N, M] (an entry counts as a one
 * when above 0.5) -> idx int64 [N, keep] the positions of its first keep ones, ascending, 0 past the count, and
 * cnt int64 [N] = min(ones, keep). One workgroup per row; a row's walk stops once keep ones are placed.
 */
int dsa_compact_mask(const float* sel, int N, int M, int keep, int64_t* idx, int64_t* cnt, void* stream);

/*
 * A selection in value order (trnrt/kernels/dsa_long_select.py:74-84, the vorder output of `select`): pools int64
 * [N, keep] ascending with cnt int64 [N] live and vals fp32 [N, keep] their scores -> out_pools / out_vals: the live
 * entries by score descending, equal scores by pool ascending, then pool 0 / NEG_INF. keep <= 8192; the outputs must
 * not alias the inputs.
 */
int dsa_value_order(const int64_t* pools, const int64_t* cnt, const float* vals, int N, int keep,
                    int64_t* out_pools, float* out_vals, void* stream);

/*
 * Slot attention over each row's visible tokens compacted in a kernel (trnrt/kernels/dsa_slots_c.py:416-447
 * `attend`, the arithmetic of dsa_sparse_mla_decode's row form): rows int32 [B, NS] pool rows of the cache viewed as
 * [num_slots / kp, kp rows], bias fp32 [B, NS, kp] (0 / NEG_INF; a token is visible when its bias is above
 * NEG_INF / 2). A compaction kernel lists each row's visible tokens (pool row kp + t, slot order); the attention then
 * runs over that list only (its rows + count form). A row with no visible token attends pool row 0's kp tokens,
 * all masked: their uniform mean, lse NEG_INF (the reference's compacted form fills empty entries with pool row 0).
 * q bf16 [B, H, Dqk], kv_fp8 [num_slots, Dqk] e4m3 rows, kv_scale fp32 [num_slots], out_bf16 [B, H, 512] or NULL,
 * out_f32 [B, H, 512] or NULL, lse fp32 [B, H] or NULL; workspace of dsa_slots_compact_workspace_bytes bytes (no
 * zero-fill needed).
 */
size_t dsa_slots_compact_workspace_bytes(int B, int H, int NS, int kp, int splits);
int dsa_sparse_mla_slots_compact(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                                 const int32_t* rows, const float* bias, void* out_bf16, float* out_f32, float* lse,
                                 void* workspace, size_t workspace_bytes, int B, int H, int Dqk, int NS, int kp,
                                 long long num_slots, float scale, int splits, void* stream);

/*
 * Token positions -> cache slots (trnrt/models/dsa_long.py:189-215 `slots` at kp = 1, no tail):
 * rows[b, k] = page_table[b, idx[b,k] / page_size] * page_size + idx[b,k] % page_size, bias[b, k] = 0 for
 * k < cnt[b] else NEG_INF (rows 0 there).
 */
int dsa_token_rows(const int32_t* idx, const int32_t* cnt, const int32_t* page_table, int32_t* rows, float* bias,
                   int B, int keep, int max_pages, int page_size, int num_pages, void* stream);

/*
 * The attention's slots of N queries (replaces trnrt/models/dsa_long.py:189-215 `slots` for any kpool kp; at kp 1 a
 * pool is a token): slot k < keep is the selected pool pools[n, k], attended when k < cnt[n]; slot keep is the
 * query's tail pool npool[n], whose tokens kp npool .. positions[n] are attended (none when positions[n] + 1 is a
 * multiple of kp); the slots past keep + 1 are padding (pool 0, masked).
 *   rows[n, s] = table_n[pool / ppp] * ppp + pool % ppp: the pool's row in the latent cache viewed as
 *   [slots / kp, kp R] (ppp = page_size / kp pools per page, a power of two); bias[n, s, t] = 0 for a token to
 *   attend, NEG_INF otherwise. pools int32 [N, keep], cnt / npool / positions int32 [N], table int32 [N, table_pages]
 *   or one [table_pages] shared by every query (table_shared = 1), rows int32 [N, n_slots], bias fp32
 *   [N, n_slots, kp]; n_slots >= keep + 1.
 */
int dsa_pool_slots(const int32_t* pools, const int32_t* cnt, const int32_t* npool, const int32_t* positions,
                   const int32_t* table, int table_shared, int32_t* rows, float* bias, int N, int keep, int n_slots,
                   int table_pages, int page_size, int kp, void* stream);

/*
 * A prefill chunk's selection in one call (replaces trnrt/kernels/dsa_long_select.py:494-528 `select`, its score
 * stage and its exact top-keep): the scores of dsa_indexer_prefill (q_scale null: bf16 queries q [N, Hi, 128]; keys
 * e4m3 with k_scale, or bf16 with k_scale null) or dsa_indexer_prefill_fp8 (q e4m3 [N, Hi, 128] with q_scale [N, Hi],
 * e4m3 keys), then per query the exact top-keep of its npool[n] candidates (rows longer than 32,768 in two levels, the
 * indexer writing the first level's sub-block maxima), returned as the reference returns them: pools int64 [N, keep]
 * ascending (0 past the count), cnt int64 [N], vals fp32 [N, keep] (the selected scores, NEG_INF past the count).
 * The queries go in tiles of tile_rows (0: tiles whose scores take at most 64 MiB), each tile scored, then selected
 * (the reference's per-tile device form, trnrt/kernels/dsa_long_pipe.py:15-25); tiles alternate between `stream`
 * and the library's second stream, which waits for the work enqueued on `stream` before the call and which `stream`
 * waits for after it (events), so one tile's selection overlaps the other stream's scores. scores: fp32
 * [N, score_stride] to receive every score, or null to keep only two tiles' scores, in the workspace (the
 * memory-bounded form).
 *   workspace: dsa_prefill_select_workspace_bytes(N, P, score_stride, keep, tile_rows, scores == null) bytes,
 *   zero-filled before first use (calls leave it so). Calls on one device run their enqueues one at a time.
 */
int dsa_prefill_select(const void* q, const float* q_scale, const float* w, const void* k, const float* k_scale,
                       const int32_t* npool, float* scores, int64_t* pools, int64_t* cnt, float* vals, void* workspace,
                       size_t workspace_bytes, int N, int Hi, int D, int P, int score_stride, int keep, float scale,
                       int tile_rows, void* stream);
size_t dsa_prefill_select_workspace_bytes(int N, int P, int score_stride, int keep, int tile_rows, int own_scores);

/*
 * The whole DSA decode layer step: indexer -> top-k -> sparse MLA (the order of trnrt/models/mla.py:506-528
 * `attention_long` at kp = 1; one call per step as trnrt/kernels/dsa_shell.py:2114-2321 `select2` fuses it).
 * scores/idx/cnt are the intermediates the caller may read afterwards (scores fp32 [B, score_stride], idx int32
 * [B, keep], cnt int32 [B]). On a GPU of 8 XCDs x 32 CUs with rows of at most 32,768 tokens (and the shapes the
 * one-launch kernel takes: Hi <= 64, H a multiple of 16 up to 512, pages of a power of two >= 32, score_stride a
 * multiple of 4, keep <= 256 * (512 / H)) the step is one kernel launch; otherwise it is dsa_decode_layer_chain.
 * The one launch, and the separate kernels' attention launch, are 256 workgroups of which the 32 on each XCD wait
 * for each other at XCD-local barriers: they need every one of their workgroups resident at once (one per CU, 160
 * KiB of LDS each). So these calls must not overlap one another on a GPU, whatever their workspaces and streams,
 * and no other kernel may hold CUs throughout one of them. A barrier wait is bounded (under a second); one that
 * gives up is counted in the workspace's status words, which dsa_layer_status reads: the call's outputs are then
 * unreliable, though every kernel ends normally.
 */
int dsa_decode_layer(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                     const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                     const int32_t* ctx_len, float* scores, int32_t* idx, int32_t* cnt, void* out_bf16, float* lse,
                     void* workspace, size_t workspace_bytes, int B, int Hi, int H, int max_pages, int page_size,
                     int num_pages, int score_stride, int max_len, int keep, float scale, int splits, void* stream);

/*
 * The same step as separate kernels enqueued back to back on one stream (indexer with the top-k's first-level
 * histogram fused, top-k, attention, split combine): any shape dsa_decode_layer accepts. Same arguments, results and
 * workspace.
 */
int dsa_decode_layer_chain(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                           const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                           const int32_t* page_table, const int32_t* ctx_len, float* scores, int32_t* idx,
                           int32_t* cnt, void* out_bf16, float* lse, void* workspace, size_t workspace_bytes, int B,
                           int Hi, int H, int max_pages, int page_size, int num_pages, int score_stride, int max_len,
                           int keep, float scale, int splits, void* stream);

/*
 * dsa_decode_layer without a workspace argument, allocating nothing (no counterpart in the reference: for callers
 * that cannot allocate device memory, such as code under HIP graph capture, tight serving loops or harnesses that
 * forbid hipMalloc). The workspace is the library's own scratch, a static device array of
 * DSA_NOALLOC_SCRATCH_BYTES per GPU (allocated with the library's code object on each GPU it runs on and held until
 * the process ends; its zero region kept as any workspace's: the first call on a device fills the zero region of
 * its batch size, and a call whose zero region (the barrier words and its rows' histograms) reaches past the
 * previous call's gets the difference filled on `stream` first, so calls of any batch sizes follow each other). A
 * call whose
 * dsa_workspace_bytes(DSA_WS_LAYER, B, H, keep, max_len, splits) exceeds that size returns DSA_ESCRATCH before any
 * HIP call. Every call on a GPU shares that GPU's scratch: calls that overlap on one GPU (several streams, host
 * threads) race and must be serialised by the caller. Arguments and results as dsa_decode_layer.
 */
#define DSA_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int dsa_decode_layer_noalloc(const void* q_idx_bf16, const float* w, const uint8_t* k_fp8, const float* k_scale,
                             const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                             const int32_t* page_table, const int32_t* ctx_len, float* scores, int32_t* idx,
                             int32_t* cnt, void* out_bf16, float* lse, int B, int Hi, int H, int max_pages,
                             int page_size, int num_pages, int score_stride, int max_len, int keep, float scale,
                             int splits, void* stream);

/*
 * Absorbed MLA over a pooled selection (replaces trnrt/models/dsa_long.py:189-215 `slots` + :218-223 `attend`
 * without materialising the slots): for each of B queries, the kp tokens of each selected pool (pools int32
 * [B, keep] ascending, cnt int32 [B] valid) and the tail tokens kp npool .. positions[b] of its incomplete pool
 * (npool int32 [B] = (positions + 1) / kp), read through page_table int32 [B, max_pages] from kv e4m3fn
 * [num_pages page_size, Dqk] with kv_scale fp32 per token; q bf16 [B, H, Dqk] (Dqk 576 or 512), out bf16 or fp32
 * [B, H, 512], lse fp32 [B, H] or null. workspace: dsa_sparse_mla_pooled_workspace_bytes(B, H, keep, kp, splits).
 */
int dsa_sparse_mla_pooled(const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale, const int32_t* pools,
                          const int32_t* cnt, const int32_t* npool, const int32_t* positions, const int32_t* page_table,
                          void* out_bf16, float* out_f32, float* lse, void* workspace, size_t workspace_bytes, int B,
                          int H, int Dqk, int keep, int kp, int max_pages, int page_size, int num_pages, float scale,
                          int splits, void* stream);
size_t dsa_sparse_mla_pooled_workspace_bytes(int B, int H, int keep, int kp, int splits);

/*
 * The pooled (GLM, kpool kp > 1) DSA decode layer step (the decode batch of
 * trnrt/models/mla.py:505-526 `attention_long`, scoring the pool-key cache's page rows in place as
 * trnrt/models/mla.py:615-630 does): the pooled indexer over the complete pools p < npool[b] of the bf16 pool-key
 * cache -> the exact top-keep pools -> sparse MLA over the kp tokens of each selected pool and the tail tokens
 * kp npool .. positions[b] of the row's incomplete pool (trnrt/models/dsa_long.py:189-223).
 *   q_idx bf16 [B, Hi, 128]; w fp32 [B, Hi] (head weights with 128 ** -0.5 folded in); pool_key bf16
 *   [num_pages page_size, 128 / kp] (pool j of page g at page row g, pool (j mod page_size / kp)); q bf16 [B, H, Dqk];
 *   kv e4m3fn [num_pages page_size, Dqk] with kv_scale fp32 per token; page_table int32 [B, max_pages]; npool int32
 *   [B] = (positions + 1) / kp; positions int32 [B]. Outputs: scores fp32 [B, max_pages page_size / kp], pools int32
 *   [B, keep] (ascending, 0 past cnt), cnt int32 [B], out bf16 [B, H, 512], lse fp32 [B, H] (or null).
 *   workspace: dsa_pooled_workspace_bytes(B, H, keep, max_pages page_size / kp, kp, splits) bytes, zero-filled
 *   before first use (calls leave the regions that must start at zero at zero). kp a power of two in [2, 8] dividing
 *   page_size; Hi <= 64; H a multiple of 16; Dqk 512 or 576. On a GPU of 8 XCDs x 32 CUs, with splits 0, Dqk 512,
 *   Hi <= 32, rows of at most 8,192 pools (max_pages page_size / kp, a multiple of 4), pages of at least 16 pools
 *   and keep kp <= 4096 / (H / 32) (H a multiple of 32), the step is one kernel launch per 8 rows (the indexer,
 *   the selection, the attention and the combine; XCD-local barriers, as dsa_decode_layer's one launch: the same
 *   co-residency rule and status words). Otherwise it is dsa_pooled_decode_layer_chain.
 */
int dsa_pooled_decode_layer(const void* q_idx_bf16, const float* w, const void* pool_key_bf16, const void* q_bf16,
                            const uint8_t* kv_fp8, const float* kv_scale, const int32_t* page_table,
                            const int32_t* npool, const int32_t* positions, float* scores, int32_t* pools,
                            int32_t* cnt, void* out_bf16, float* lse, void* workspace, size_t workspace_bytes, int B,
                            int Hi, int H, int Dqk, int max_pages, int page_size, int num_pages, int kp, int keep,
                            float scale, int splits, void* stream);

/*
 * The same pooled step as separate kernels enqueued back to back on one stream: the pooled indexer with the top-k's
 * first-level histogram fused, the top-keep pools, then (splits 0, Dqk 512, H a multiple of 32 and the token slots
 * in 128-slot splits) the attention and combine as one XCD-local launch, otherwise the split attention and the
 * combine kernel. Any shape dsa_pooled_decode_layer accepts; same arguments, results and workspace.
 */
int dsa_pooled_decode_layer_chain(const void* q_idx_bf16, const float* w, const void* pool_key_bf16,
                                  const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                                  const int32_t* page_table, const int32_t* npool, const int32_t* positions,
                                  float* scores, int32_t* pools, int32_t* cnt, void* out_bf16, float* lse,
                                  void* workspace, size_t workspace_bytes, int B, int Hi, int H, int Dqk,
                                  int max_pages, int page_size, int num_pages, int kp, int keep, float scale,
                                  int splits, void* stream);

/*
 * The pooled decode step: the pool-key write of the step's written tokens (one per row, at positions[b], cache slot
 * slot_mapping[b]; dsa_pool_keys_write's arithmetic and arguments, with n_rows = B and the layer's page_size and
 * num_pages page_size slots) followed by dsa_pooled_decode_layer on the written cache, as the reference's decode
 * step runs them (trnrt/models/mla.py:448-452: write_pool_keys, then attention_long). Where dsa_pooled_decode_layer
 * is one launch and kp is 4, so is this: the workgroup whose block holds a row's written pool computes the pool's
 * key, stores it, and scores that pool (when it is complete) from the new key, so scores, selection and outputs equal
 * the write followed by the layer. Otherwise it is dsa_pool_keys_write then dsa_pooled_decode_layer. pool_key is
 * written (the written pools' slots) and read; other arguments, results and workspace as dsa_pooled_decode_layer.
 */
int dsa_pooled_decode_step(const void* rows, int rows_fp8, const float* rows_scale, int rows_width, const float* ape,
                           const int64_t* slot_mapping, const void* q_idx_bf16, const float* w, void* pool_key_bf16,
                           const void* q_bf16, const uint8_t* kv_fp8, const float* kv_scale,
                           const int32_t* page_table, const int32_t* npool, const int32_t* positions, float* scores,
                           int32_t* pools, int32_t* cnt, void* out_bf16, float* lse, void* workspace,
                           size_t workspace_bytes, int B, int Hi, int H, int Dqk, int max_pages, int page_size,
                           int num_pages, int kp, int keep, float scale, int splits, void* stream);

/* Bytes of workspace dsa_pooled_decode_layer needs (max_len: the most pools a row scores). */
size_t dsa_pooled_workspace_bytes(int B, int H, int keep, int max_len, int kp, int splits);

/*
 * Quantise-on-write of n_rows rows into a paged FP8 cache, the cache-store step before the path (replaces
 * trnrt/models/decoder.py:481-486 `_store`, which trnrt/models/mla.py:445-446 calls for the latent rows and the
 * indexer-key rows at slot_mapping):
 *   x: bf16 [n_rows, W] (x_fp32 = 0) or fp32 [n_rows, W] (x_fp32 = 1); slots int64 [n_rows] (cache slots
 *   table[pos / page_size] * page_size + pos % page_size, trnrt/models/decoder.py:658-667); cache uint8 e4m3fn
 *   [num_slots, W]; scale fp32 [num_slots] or null.
 *   per_token_scale = 1 (this build's format; scale required): s = max(absmax(row), 1e-30) / 448,
 *     cache[slot] = e4m3fn(clamp(row / s, +-fp8_max)), scale[slot] = s;
 *   per_token_scale = 0 (the reference's form, KV scale 1.0): cache[slot] = e4m3fn(clamp(row, +-fp8_max)),
 *     scale[slot] = 1 when a scale array is given.
 *   fp32 arithmetic with a correctly rounded division, round-to-nearest-even into e4m3fn (torch's cast).
 *   W a multiple of 8 in [8, 1024]; 0 < fp8_max <= 448. A row whose slot is outside [0, num_slots) is not written;
 *   rows that share a slot leave one of them (unspecified which).
 */
int dsa_cache_write(const void* x, int x_fp32, const int64_t* slots, uint8_t* cache, float* scale, int n_rows, int W,
                    long long num_slots, int per_token_scale, float fp8_max, void* stream);

/*
 * GLM's pooled indexer keys, written with the cache (replaces trnrt/models/mla.py:1277-1296 `write_pool_keys`, with
 * trnrt/models/glm5_next.py:151-160 `pool_keys` and the slots of mla.py:1262-1274 `_pool_key_slots`): for each of
 * n_rows written tokens, the pool of kp tokens it belongs to (positions first .. first + kp - 1, first = pos - pos % kp)
 * gets the key
 *   pk[d] = bf16(sum_t bf16(bf16(softmax_t(g_t[d] + ape[t, d])) * k_t[d])),  d < 128  (softmax over the pool in fp32)
 * from the pool's cached indexer rows [key k (128) | gate logits g (128)], written as kp pieces of 128 / kp values,
 * piece i into the slot of the pool's i-th token. A padded row (slot_mapping < page_size: the null page) reads and
 * writes its own slot only. A pool lies inside one page (kp divides page_size), so the slots of its tokens, which the
 * reference looks up through the page table, are slot_mapping[row] - pos % kp + t: page_table (int32 [n_rows,
 * table_pages] or one shared [table_pages], table_shared = 1) is taken for the reference's signature, may be null,
 * and is not read.
 *   rows [num_slots, rows_width]: e4m3fn (rows_fp8 = 1; with rows_scale fp32 [num_slots] the per-token scale, or null
 *   for the reference's unscaled cache; read as bf16 values) or bf16; ape fp32 [kp, 128]; positions int32 [n_rows];
 *   slot_mapping int64 [n_rows]; pool_key bf16 [num_slots, 128 / kp]. kp a power of two <= 8 dividing page_size; rows_width >= 256.
 */
int dsa_pool_keys_write(const void* rows, int rows_fp8, const float* rows_scale, int rows_width, const float* ape,
                        const int32_t* positions, const int32_t* page_table, int table_shared, int table_pages,
                        const int64_t* slot_mapping, void* pool_key, int n_rows, int kp, int page_size,
                        long long num_slots, void* stream);

/*
 * Bytes of workspace an entry point needs. kind: DSA_WS_TOPK (B, max_len, keep), DSA_WS_ATTENTION (B, H, keep,
 * splits; splits 0 = the GPU default), DSA_WS_LAYER (all of them). Unused arguments are ignored.
 */
size_t dsa_workspace_bytes(int kind, int B, int H, int keep, int max_len, int splits);

/* The split count dsa_sparse_mla_decode uses for splits = 0. */
int dsa_default_splits(int B, int H, int keep);

/*
 * The status words of a decode workspace (no counterpart in the reference, whose device kernels never report and
 * whose host wrappers raise, trnrt/kernels/dsa_index.py:258-259): what the calls since the last clear counted,
 * summed over the XCDs. *gave_up: barrier waits of dsa_decode_layer (one launch), dsa_decode_layer_chain's attention
 * launch or dsa_pooled_decode_layer's attention launch that gave up (non-zero: some of those calls' outputs may be
 * wrong); *two_exchange: rows the one-launch layer selected in its two-exchange form (statistics). workspace: a
 * decode workspace, or NULL for the current device's dsa_decode_layer_noalloc scratch. Synchronises `stream` (the
 * only entry point that does), and with clear != 0 zeroes the counts (a fill kernel on `stream`, then a second
 * synchronisation); must not overlap a call on the same workspace. Returns DSA_OK, DSA_EINVAL or DSA_ELAUNCH.
 */
int dsa_layer_status(void* workspace, int32_t* gave_up, int32_t* two_exchange, int clear, void* stream);

/*
 * Kernel timing for benchmarks (no counterpart in the reference, whose kernels are timed by the Neuron profiler).
 * Between dsa_timing_begin and dsa_timing_end on one host thread, the k-th kernel the library launches records
 * events[2k] and events[2k+1] (hipEvent_t values created by the caller) at the kernel's own start and end, for
 * k < pairs; dsa_timing_end returns how many kernels were launched and dsa_timing_kernel_name(k) names the k-th
 * (valid until the next dsa_timing_begin on the thread).
 */
int dsa_timing_begin(void* const* events, int pairs);
int dsa_timing_end(void);
const char* dsa_timing_kernel_name(int k);

#ifdef __cplusplus
}
#endif

#endif /* DSA_GFX950_H */
