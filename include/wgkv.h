/*
 * wgkv.h -- C ABI of the MI355X write-gated dual-cache KV path.
 *
 * Every entry point takes raw device pointers, element strides and sizes and
 * a hipStream_t (passed as void*), enqueues its kernels on that stream and
 * returns a status code.  Nothing here allocates or frees caller memory;
 * kernels that need scratch take a caller-provided workspace whose size is
 * reported by the matching *_workspace_bytes function.  No entry point
 * synchronises with the host.
 *
 * Tensor dtypes: "bf16" is IEEE bfloat16 stored as uint16, "i32" int32,
 * "u8" one byte per boolean (0/1), "f32" float32.
 */
#ifndef WGKV_H_
#define WGKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define WGKV_OK 0
#define WGKV_ERR_ARG 1          /* inconsistent or out-of-range argument      */
#define WGKV_ERR_UNSUPPORTED 2  /* shape/dtype the kernels are not built for   */
#define WGKV_ERR_CAPACITY 3     /* cache capacity would be exceeded            */
#define WGKV_ERR_WORKSPACE 4    /* workspace missing or too small              */
#define WGKV_ERR_HIP 5          /* a HIP runtime call failed                   */

/* Library version, for the Python loader's sanity check. */
int wgkv_version(void);

/* Human-readable text of a status code (static storage). */
const char* wgkv_status_string(int status);

/* ------------------------------------------------------------------------
 * Ragged paged decode attention over the dual cache.
 *
 * Replaces the reference's decode kernel handle
 *   flash_attn_with_kvcache_wrapper_triton_handle   src/modeling_layers.py:1007-1136
 *   (split kernel :834-943, reduce kernel :946-1000, host planner :1024-1069)
 * and its alternative flash_attn_with_kvcache_wrapper :766-811, with the
 * contract of decode_kernel_handle at :1439-1447:
 *   q            bf16 (B, Hq, D)          element strides q_stride_b, q_stride_h; d contiguous
 *   k_cache/v_cache bf16 (num_pages, page_size, D), contiguous
 *   cache_seqlens i32 (B, Hkv)            stride sl_stride_b; h contiguous
 *   block_table  i32 (B, Hkv, max_pages)  strides bt_stride_b, bt_stride_h; contiguous pages
 *   out          bf16 (B, Hq, D)          strides out_stride_b, out_stride_h
 * For every (b, h_kv) the first cache_seqlens[b,h] tokens of the logical
 * sequence (page i of the head = block_table[b,h,i]) are attended by the
 * Hq/Hkv query heads h_kv*G .. h_kv*G+G-1 with softmax(q.k * scale) v.  A head
 * with zero tokens yields zeros.  Supported: D in {64,128}, page_size in
 * {16,32,64}, G = Hq/Hkv in 1..8, B*Hkv <= 2048.  Split planning happens
 * on the device; out-of-range lengths are clamped to max_pages*page_size and
 * out-of-range page ids to the pool, so no access leaves the buffers.  With
 * B*Hkv < 32 and G <= 4 a call is one kernel launch (the split partials of a
 * head are merged by its last chunk to finish); otherwise it is two, the
 * split kernel and a merge kernel.
 * The workspace (wgkv_paged_decode_workspace_bytes) holds per-head arrival
 * counters and the split partials: zero-fill it before its first call; every
 * call leaves the counters zero again.  Calls that share a workspace must be
 * ordered (one stream, or events between streams).
 * ---------------------------------------------------------------------- */
size_t wgkv_paged_decode_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t head_dim);

int wgkv_paged_decode_attn(
    const void* q, int64_t q_stride_b, int64_t q_stride_h,
    const void* k_cache, const void* v_cache, int64_t num_pages, int32_t page_size,
    const int32_t* cache_seqlens, int64_t sl_stride_b,
    const int32_t* block_table, int64_t bt_stride_b, int64_t bt_stride_h, int32_t max_pages,
    void* out, int64_t out_stride_b, int64_t out_stride_h,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale,
    void* workspace, size_t workspace_bytes,
    void* stream);

/* Allocation-free form of wgkv_paged_decode_attn.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory or
 * pass a workspace (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * wgkv_paged_decode_attn minus the workspace; the arrival counters and split
 * partials live in a static device array of the library (12.2 MiB per device,
 * held until the process ends) that covers every supported call (head_dim <=
 * 128, G <= 8, batch*num_kv_heads <= 2048; larger sizes return
 * WGKV_ERR_UNSUPPORTED).  The array's device address is looked up on the
 * first call on each device, which also zeroes the counters with a small
 * kernel on the call's stream; every call leaves them zero.  All calls on
 * one device share the array: calls that overlap on one GPU (different
 * streams, no ordering between them) race and must not be made. */
int wgkv_paged_decode_attn_noalloc(
    const void* q, int64_t q_stride_b, int64_t q_stride_h,
    const void* k_cache, const void* v_cache, int64_t num_pages, int32_t page_size,
    const int32_t* cache_seqlens, int64_t sl_stride_b,
    const int32_t* block_table, int64_t bt_stride_b, int64_t bt_stride_h, int32_t max_pages,
    void* out, int64_t out_stride_b, int64_t out_stride_h,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, void* stream);

/* ------------------------------------------------------------------------
 * Vertical-slash metadata of the sparse prefill, built on the device.
 *
 * Replaces generate_sparse_indices (src/modeling_layers.py:384-409) with its
 * helpers generate_block_offset (:321-349) and generate_column_index
 * (:352-381); same outputs, no host synchronisation:
 *   g_mask        u8 (B, Hkv, S)  strides gm_stride_b, gm_stride_h; s contiguous
 *   block_count   i32 (R)          R = ceil(S / block)
 *   block_offset  i32 (R, P+1)     P = min(W / block, R)
 *   column_count  i32 (B, Hkv, R)  admitted positions < r*block - W + 1 (0 for r < P)
 *   column_index  i32 (B, Hkv, col_cap)  admitted positions < 1 + block*((S-1)/block),
 *                                  ascending; entries past a head's count are unspecified
 *   column_total  i32 (B, Hkv) or NULL: number of listed positions per head
 * The reference sizes column_index to the largest per-head count (a host
 * sync); here the caller passes col_cap (S always suffices) and positions past
 * col_cap are dropped.  W must be a multiple of block (reference :394).
 * ---------------------------------------------------------------------- */
int wgkv_build_prefill_meta(
    const uint8_t* g_mask, int64_t gm_stride_b, int64_t gm_stride_h,
    int32_t batch, int32_t num_kv_heads, int32_t seq_len, int32_t local_window, int32_t block,
    int32_t* block_count, int32_t* block_offset,
    int32_t* column_count, int32_t* column_index, int32_t col_cap, int32_t* column_total,
    void* stream);

/* ------------------------------------------------------------------------
 * Dual cache: pool of total_pages pages of page_size rows of head_dim bf16,
 * one pool for K and one for V (reference layout, src/modeling_layers.py:
 * 1209-1216).  Local pages of (layer l, head h) are the first W/page entries
 * of block_table[l][h] and hold ring slot s at pool row (l*H + h)*W + s
 * (:1265-1271, :1282-1284).  block_table is (L, H, max_pages_per_head)
 * contiguous, global_lengths (L, H), local_is_global u8 (L, H, W),
 * local_pre_key bf16 (L, H, W, D) or NULL, next_free_block a device int32.
 * On a capacity failure nothing is written and *status = WGKV_ERR_CAPACITY
 * (the caller reads status when it needs to raise).
 * ---------------------------------------------------------------------- */

/* Prefill admission of one layer, batch 1 (the reference's inference batch,
 * :1614).  Replaces the local-ring write (:1290-1300) and the per-head global
 * scatter loop (:1302-1331) of prefill_wrapper:
 *   key/value   bf16 (H, S, D)  strides kv_stride_h, kv_stride_s; d contiguous
 *   pre_key     bf16 (H, S, D)  or NULL (stored in local_pre_key when given)
 *   g_mask      u8 (H, S)       admission flags (g > threshold)
 * Admitted positions of [0, S-W) are compacted in ascending order into fresh
 * contiguous pages bump-allocated in head order from *next_free_block; the
 * last min(S, W) positions fill ring slots 0.. with their flags.  Capacity:
 * min(S,W) + admitted <= max_tokens_per_head per head with admissions, and
 * the pages fit in total_pages (:1312-1321). */
size_t wgkv_prefill_admit_workspace_bytes(int32_t num_kv_heads, int32_t seq_len);

int wgkv_prefill_admit(
    const void* key, const void* value, int64_t kv_stride_h, int64_t kv_stride_s,
    const void* pre_key, int64_t pk_stride_h, int64_t pk_stride_s,
    const uint8_t* g_mask, int64_t gm_stride_h,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t seq_len, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* status,
    void* workspace, size_t workspace_bytes, void* stream);

/* Decode-step cache update.
 * do_migrate: lazy promotion, replacing migrate_local_kv_to_global (:674-763):
 *   ring slot local_ptr of every (layer, head) flagged in local_is_global is
 *   appended to that head's global pages; a new page is bump-allocated when
 *   the global length is a multiple of page_size, in row-major (layer, head)
 *   order; capacity W + len + 1 <= max_tokens_per_head and total_pages.
 * do_write: the ring write of decode_wrapper (:1390-1413) for `layer`:
 *   key/value bf16 (H, D) (stride kv_stride_h) go to slot local_length if the
 *   ring is filling, else local_ptr; g_mask u8 (H) sets the slot's flag, or,
 *   if g_mask is NULL (deferred gating), pre_key (H, D) is stored in
 *   local_pre_key; cache_seqlens i32 (H) (may be NULL) receives
 *   min(local_length+1, W) + global_lengths[layer] (:1429-1432).
 * local_ptr / local_length are the host-side ring state before this step.
 * quest_key_min / quest_key_max: the QUEST page key bounds, bf16
 * (total_pages, D), or both NULL; a promoted token starts its page's bounds
 * (first row) or widens them (src/modeling_layers.py:744-761).
 * free_ids / free_count: SnapKV's list of released pages (i32, ids in
 * release order, and its device length) or both NULL; pages for promotion
 * come from the last entries of the list first, in list order, then from
 * next_free_block (:694-712). */
int wgkv_decode_append(
    const void* key, const void* value, int64_t kv_stride_h,
    const void* pre_key, int64_t pk_stride_h,
    const uint8_t* g_mask,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    int32_t local_ptr, int32_t local_length, int32_t do_migrate, int32_t do_write,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* cache_seqlens, int32_t* status,
    void* quest_key_min, void* quest_key_max, int32_t* free_ids, int32_t* free_count,
    void* stream);

/* wgkv_decode_append with the ring state in device memory, int32[3] =
 * (local_ptr, local_length, slot of the last ring write), instead of host
 * arguments, for decode steps replayed from a captured HIP graph: promotion
 * runs only if the device local_length equals W (the host condition of
 * :1470); a ring write stores its slot in ring_state[2] (deferred gating
 * re-gates the window when that slot is W-1, :1402-1405); with advance != 0
 * (the last layer's call) the kernel advances the ring state as
 * decode_wrapper's host update does (:1409-1413).  Same arguments
 * otherwise. */
int wgkv_decode_append_ring(
    const void* key, const void* value, int64_t kv_stride_h,
    const void* pre_key, int64_t pk_stride_h,
    const uint8_t* g_mask,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    int32_t* ring_state, int32_t advance, int32_t do_migrate, int32_t do_write,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* cache_seqlens, int32_t* status,
    void* quest_key_min, void* quest_key_max, int32_t* free_ids, int32_t* free_count,
    void* stream);

/* Random admission flags (the random_sparsity ablation).
 *
 * Replaces get_random_g_scores (src/modeling_layers.py:1160-1166) where a
 * decode step uses it: the deferred window refresh (:1177-1178) and the
 * per-token scores of a decode step.  flags u8 (num_kv_heads, n) with row
 * stride flags_stride_h: flags[h][i] = r >= bf16(random_sparsity) for a
 * draw r in [0, 1) (a token is admitted iff its score, 1 or 0, exceeds
 * g_threshold; so random_sparsity 0 admits every token and 1 none).  The
 * draws come from a counter-based generator keyed by (seed, *draw_counter,
 * h, i); each call that runs advances *draw_counter (a device int32) by one,
 * so eager calls and replays of a captured call continue one sequence.  With
 * active_flag != NULL the call does nothing unless *active_flag ==
 * active_value (decided on the device).  One kernel launch; n*num_kv_heads
 * of any size. */
int wgkv_random_admission(uint8_t* flags, int64_t flags_stride_h, int32_t num_kv_heads, int32_t n,
                          float random_sparsity, uint64_t seed, int32_t* draw_counter,
                          const int32_t* active_flag, int32_t active_value, void* stream);

/* ------------------------------------------------------------------------
 * Write-gate scores and admission flags.
 *
 * Replaces GatingPredictor.forward (src/modeling_layers.py:170-205) with its
 * GatingRMSNorm inputs (:113-131) and the admission test g > g_threshold
 * (:1465, :1180).  Inputs (B, H, S, D) with per-input strides, d contiguous,
 * dtype bf16 (in_dtype 0) or f32 (1); inputs_mask bit 0/1/2 selects pre_k /
 * post_k / v (concatenated in that order, :173-183).  Weights f32 with the
 * reference's state-dict shapes: norm weights (D); w1 = conv1.weight
 * (H*inner, n_in*D); b1 (H*inner); w2 = conv2.weight (H, inner); b2 (H).
 * With rms != 0 each input row is x*rsqrt(mean(x^2)+1e-6), cast to the input
 * dtype, times its norm weight.  act 0 = exact-erf GELU, 1 = SiLU.
 * clamp_min > 0 applies the conv path's clamp (:205).  Outputs (may be NULL,
 * not both): scores f32 (B,H,S), mask u8 (B,H,S) = scores > threshold.
 * precision: 0 = the gate with fp32 parameters (fp32 arithmetic after the
 * inputs' norm cast); 1 / 2 = the gate with bf16 parameters, the reference's
 * inference configuration (its scripts load the gate checkpoint in bf16,
 * scripts/profiling.py:222-226), on bf16 inputs: each op's result is rounded
 * to bf16 as torch rounds it -- the norm product, the first layer (1 = fast
 * path :186-190: einsum output rounded, then the bias add rounded; 2 = conv
 * path :197-199: one rounding after the bias), the activation, the second
 * layer likewise, the sigmoid -- the weights passed as f32 copies of the
 * bf16 values, and the score is compared with bf16(threshold) and clamped
 * to bf16(clamp_min), as a bf16 tensor compared with a Python float is.
 * Supported: D in {64,128}, inner a multiple of 16, n_in*D <= 384.
 * w1_packed (may be NULL): the same weights as written by
 * wgkv_gate_pack_weights with the same precision.  With bf16 inputs (16-byte
 * aligned, strides multiples of 8 elements; with precision != 0 16-byte
 * aligned norm weights) and seq_len > 4 the first layer then runs on the
 * bf16 matrix core.  precision 0: the norm weights are folded into w1 in
 * fp32 and the product split into three bf16 planes that carry all its
 * bits, so the result equals the fp32 layer up to rounding order; precision
 * 1 / 2: one plane, w1 itself.  Otherwise ignored (w1 and the norm weights
 * are always read by the other paths).
 * active_flag (may be NULL): a device int32; when given, the launch does
 * nothing unless *active_flag == active_value -- the condition is read on the
 * device, so a captured decode step can re-gate its window only on the step
 * that fills the ring's last slot (deferred gating, :1402-1405).
 * workspace (may be NULL): for seq_len <= 4 (decode steps) the hidden
 * columns of each head are split over several workgroups whose partial
 * logits meet in the workspace; it must hold wgkv_gate_workspace_bytes()
 * bytes, be zero-filled before its first use and not be shared by
 * concurrent calls (each call leaves its counters at zero again).  With
 * NULL one workgroup per head takes all columns.
 * ---------------------------------------------------------------------- */
int64_t wgkv_gate_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t inner);
int wgkv_gate_scores(
    const void* pre_key, int64_t pk_sb, int64_t pk_sh, int64_t pk_ss,
    const void* post_key, int64_t k_sb, int64_t k_sh, int64_t k_ss,
    const void* value, int64_t v_sb, int64_t v_sh, int64_t v_ss,
    int32_t in_dtype, int32_t inputs_mask,
    const float* w_pre, const float* w_post, const float* w_v,
    const float* w1, const float* b1, const float* w2, const float* b2,
    int32_t batch, int32_t num_kv_heads, int32_t seq_len, int32_t head_dim, int32_t inner,
    int32_t act, int32_t rms, int32_t precision, float clamp_min, float threshold,
    float* scores, int64_t sc_sb, int64_t sc_sh,
    uint8_t* mask, int64_t mk_sb, int64_t mk_sh,
    const void* w1_packed,
    const int32_t* active_flag, int32_t active_value,
    void* workspace, int64_t workspace_bytes,
    void* stream);

/* Packed first-layer weights of the gate (no reference counterpart: a
 * one-time layout of GatingPredictor's conv1.weight and norm weights,
 * src/modeling_layers.py:134-161, for the bf16 matrix-core path above).
 * wgkv_gate_packed_bytes: size for in_features = n_in * head_dim (a multiple
 * of 32) and inner (a multiple of 16), or -1.  wgkv_gate_pack_weights writes,
 * for precision 0, w_norm_i[d] * w1[h*inner + j][i*D + d] (norm weights only
 * with rms != 0) as three bf16 planes hi + mid + lo; for precision 1 / 2,
 * w1 as one bf16 plane (its values are bf16; the norm weights are applied
 * to the inputs).  inputs_mask, rms and precision as for wgkv_gate_scores.
 * Repack after the weights change. */
int64_t wgkv_gate_packed_bytes(int32_t num_kv_heads, int32_t inner, int32_t in_features, int32_t precision);
int wgkv_gate_pack_weights(
    const float* w_pre, const float* w_post, const float* w_v, int32_t inputs_mask, int32_t rms,
    const float* w1, int32_t num_kv_heads, int32_t head_dim, int32_t inner, int32_t precision,
    void* packed, int64_t packed_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Sparse (vertical-slash) causal prefill attention.
 *
 * Replaces the external sparse_attn_func called by prefill_wrapper
 * (src/modeling_layers.py:1366-1374; contract pinned by
 * utils/test_sparse_attn.py:34-93):
 *   q   bf16 (B, S, Hq, D)   strides q_sb, q_ss, q_sh; d contiguous
 *   k,v bf16 (B, S, Hkv, D)  strides kv_sb, kv_ss, kv_sh
 *   out bf16 (B, S, Hq, D)   strides o_sb, o_ss, o_sh
 *   metadata as produced by wgkv_build_prefill_meta (block = 64):
 *   block_count (R), block_offset (R, block_offset_width), column_count
 *   (B, Hkv, R) contiguous, column_index with strides ci_sb, ci_sh.
 * Row block r of head hq (KV head hq / G) attends to the listed admitted
 * columns and to the band blocks [o, o+64), causally.  Softmax in fp32.
 * Supported: D in {32,64,128}, G = Hq/Hkv from 1 to 8, block 64.
 * ---------------------------------------------------------------------- */
int wgkv_sparse_prefill_attn(
    const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    const void* k, const void* v, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
    void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    const int32_t* block_count, const int32_t* block_offset, int32_t block_offset_width,
    const int32_t* column_count, const int32_t* column_index, int64_t ci_sb, int64_t ci_sh,
    int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block, float softmax_scale, void* stream);

/* ------------------------------------------------------------------------
 * Chunked gated prefill (batch 1): the prompt goes in chunks
 * [chunk_start, chunk_start + chunk_len) and each chunk leaves the dual cache
 * as a one-shot prefill of the first chunk_start + chunk_len tokens would
 * (wgkv_prefill_admit; reference prefill_wrapper, src/modeling_layers.py:
 * 1183-1300), the same logical cache per head -- (position, K, V) in order --
 * with pages numbered in chunk order.  The reference prefills in one call
 * (:1197 asserts a single initialisation); these two entry points extend
 * that call for prompts fed in pieces.  Per chunk and layer:
 *   1. wgkv_chunk_cache_update(stage 0): admission of positions
 *      [chunk_start - W, chunk_start + chunk_len - W) -- the previous ring
 *      (slot i = position chunk_start - W + i, flags in local_is_global)
 *      then the chunk's own -- appended in position order to each head's
 *      global pages (bump-allocated in head order); column_count (Hkv, R_c)
 *      of the chunk's R_c = ceil(chunk_len/64) row blocks = admitted
 *      positions below max(0, 64 r - W + 1), r the global row block.
 *   2. wgkv_chunk_prefill_attn: the vertical-slash attention of the
 *      chunk's queries (the masks of utils/test_sparse_attn.py:34-58 at the
 *      chunk's rows): admitted columns through the head's block table, band
 *      keys below chunk_start from the ring, the rest from the chunk.
 *   3. wgkv_chunk_cache_update(stage 1): ring slot i <- position
 *      chunk_start + chunk_len - W + i (flags and, with pre_key, the
 *      deferred-gating pre-RoPE keys); the global lengths and
 *      next_free_block take the chunk's admissions here.
 * Stage 0 is one launch (counts, plan and compaction); the pages and block
 * table entries are final after it, the lengths after stage 1.  Both stages
 * of one chunk take the same workspace (stage 0 leaves the counts and an
 * abort flag there that stage 1 reads: a capacity failure sets status =
 * WGKV_ERR_CAPACITY and the chunk writes nothing).  Up to 1024 heads.  key/value/pre_key are the
 * chunk's (Hkv, chunk_len, D) bf16 (strides per head and per position, d
 * contiguous); g_mask (Hkv, chunk_len) u8.  Requires chunk_start and W
 * multiples of 64, W a multiple of page_size and, after the first chunk,
 * chunk_start >= W and chunk_len >= W.
 * ---------------------------------------------------------------------- */
size_t wgkv_chunk_admit_workspace_bytes(int32_t num_kv_heads, int32_t chunk_len, int32_t local_window);

int wgkv_chunk_cache_update(
    int32_t stage,
    const void* key, const void* value, int64_t kv_stride_h, int64_t kv_stride_s,
    const void* pre_key, int64_t pk_stride_h, int64_t pk_stride_s,
    const uint8_t* g_mask, int64_t gm_stride_h,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t chunk_start, int32_t chunk_len, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* status, int32_t* column_count,
    void* workspace, size_t workspace_bytes, void* stream);

/* q (chunk_len, Hq, D) and out with strides q_ss/q_sh, o_ss/o_sh; the
 * chunk's k/v (chunk_len, Hkv, D) with strides kv_ss/kv_sh; pool_k/pool_v
 * (pages*page_size, D) and block_table (L, Hkv, max_pages_per_head) of the
 * cache, column_count (Hkv, R_c) from stage 0.  Supported: D in {32,64,128},
 * G = Hq/Hkv in 1..8, page_size 16, 32 or 64 (the reference's block_size,
 * 16 by default, :1209-1216; a page must divide the kernel's 64-key tile). */
int wgkv_chunk_prefill_attn(
    const void* q, int64_t q_ss, int64_t q_sh,
    const void* k, const void* v, int64_t kv_ss, int64_t kv_sh,
    void* out, int64_t o_ss, int64_t o_sh,
    const void* pool_k, const void* pool_v,
    const int32_t* block_table, int32_t max_pages_per_head,
    const int32_t* column_count,
    int32_t layer, int32_t chunk_start, int32_t chunk_len,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, float softmax_scale, void* stream);

/* ------------------------------------------------------------------------
 * QUEST page selection over the dual cache (the reference's comparison
 * baseline, src/modeling_layers.py:452-576; bounds kept at :1333-1347 and
 * :744-761).  key_min / key_max: bf16 (total_pages, D), one row per pool page.
 *
 * wgkv_quest_update_bounds: for every head of `layer`, recompute the bounds
 * of the logical global pages [from/page, ceil(len/page)) -- from =
 * from_lengths[h] (i32 (H), the global lengths before the update) or 0 when
 * from_lengths is NULL -- as the elementwise min / max of the page's valid
 * key rows (what the reference's prefill writes and its decode-time updates
 * accumulate).  Call after wgkv_prefill_admit (from NULL) or after a chunk's
 * admission (from = the lengths before it).
 *
 * wgkv_quest_select: the selection of quest_select_blocks for one decode
 * step of `layer`: q bf16 (Hq, D) (stride q_stride_h) of the step's token;
 * each KV head scores its full global pages by max over its G query heads of
 * sum_d q_d * (q_d >= 0 ? key_max_d : key_min_d) (fp32; with scores_bf16
 * != 0 rounded as the reference's bf16 torch ops round it: each product to
 * bf16, the fp32 sum to bf16), keeps the top
 * k = min(ceil(max(budget - local_tokens, 0)/page), global pages) - (1 if a
 * partial page exists) full pages (equal scores at the cut: lowest page
 * first) and the partial page, and writes sel_block_table i32 (H, sel_cap):
 * the head's first ceil(local_tokens/page) local pages, the kept full pages
 * in page order, then the partial page; sel_seqlens i32 (H) = local_tokens +
 * the kept tokens.  These feed wgkv_paged_decode_attn (batch 1).  sel_cap >=
 * ceil(local_tokens/page) + ceil(max(budget - local_tokens, 0)/page).
 * ---------------------------------------------------------------------- */
int wgkv_quest_update_bounds(
    const void* pool_k, const int32_t* block_table, int32_t max_pages_per_head,
    const int32_t* global_lengths, const int32_t* from_lengths,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t local_window, int32_t page_size,
    int32_t head_dim, void* key_min, void* key_max, void* stream);

size_t wgkv_quest_select_workspace_bytes(int32_t num_kv_heads, int32_t max_pages_per_head);

int wgkv_quest_select(
    const void* q, int64_t q_stride_h,
    const int32_t* block_table, int32_t max_pages_per_head, const int32_t* global_lengths,
    const void* key_min, const void* key_max,
    int32_t layer, int32_t num_layers, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t local_tokens, int32_t token_budget, int32_t scores_bf16,
    int32_t* sel_block_table, int32_t sel_cap, int32_t* sel_seqlens,
    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * SnapKV eviction over the dual cache (the reference's comparison baseline,
 * snapkv_evict, src/modeling_layers.py:595-671, and its trigger :1500-1507),
 * in four launches with no host synchronisation.
 *
 * Runs only if the sum of global_lengths (L*H) exceeds max_cached_tokens
 * (decided on the device; state[0] = 1 when it ran, state[1] counts the
 * evictions, the reference's snapkv_evict_count).  Then, for every (layer,
 * KV head) with n global tokens and n_evict = int(n * evict_ratio) > 0: the
 * window queries query_window bf16 (L, window, Hq, D) (the reference's
 * snapkv_query_buffer, Hq = H * num_kv_groups) score the head's global keys
 * -- softmax over the keys of q.k * softmax_scale (logits_bf16 != 0: the
 * logit rounded as the reference's bf16 matmul and scalar multiply round
 * it, bf16(bf16(q.k) * scale); 0: fp32), max over the group's query heads,
 * mean over the window, max-pooled over kernel_size (odd) positions --, the
 * n_evict lowest pooled scores are dropped (equal scores: lower position
 * first; the reference's topk leaves their order unspecified), the kept
 * tokens are packed in order into the head's first pages of pool_k /
 * pool_v (bf16 (total_pages*block_size, D)), global_lengths is set to the
 * kept count, and the head's pages past the kept ones are appended to
 * free_ids (free_count entries, heads in (layer, head) order, pages in
 * table order) with their block_table entries set to total_pages - 1.
 * block_table i32 (L, H, max_pages): local_pages ring pages, then the
 * global pages.  scores_out (may be NULL): f32 (L*H, max_tokens_per_head),
 * the pooled scores of each evicted head's tokens.  D in {64, 128},
 * num_kv_groups <= 8.  workspace: wgkv_snapkv_workspace_bytes() bytes,
 * 256-byte aligned, not shared by concurrent calls.
 * ---------------------------------------------------------------------- */
int64_t wgkv_snapkv_workspace_bytes(int32_t num_layers, int32_t num_kv_heads, int32_t num_kv_groups,
                                    int32_t window, int32_t max_tokens_per_head);
int wgkv_snapkv_evict(
    void* pool_k, void* pool_v, int32_t* block_table, int32_t* global_lengths,
    int32_t* free_ids, int32_t* free_count, const void* query_window,
    int32_t num_layers, int32_t num_kv_heads, int32_t num_kv_groups, int32_t head_dim, int32_t block_size,
    int32_t local_pages, int32_t max_pages, int32_t total_pages, int32_t max_tokens_per_head,
    int32_t window, int32_t kernel_size, double evict_ratio, float softmax_scale, int64_t max_cached_tokens,
    int32_t logits_bf16, int32_t* state, float* scores_out,
    void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Decoder building blocks for the end-to-end harness around the path (bf16).
 * No counterpart among the path's functions: each replaces a chain of torch
 * kernels of the reference model with one launch, with the same bf16
 * rounding points.
 *
 * wgkv_rms_norm -- LlamaRMSNorm (src/modeling_llama.py:61-76), optionally
 *   after the residual add (:366, :399): rows of `hidden` bf16 (row strides
 *   in elements); with residual (and residual_out, may equal x) h = x +
 *   residual is stored to residual_out and normalised.  out = weight *
 *   bf16(h * rsqrt(mean(h^2) + eps)).  hidden a multiple of 8, <= 8192.
 * wgkv_rope_qkv -- apply_rotary_pos_emb (:115-146) for q (B,S,Hq,D) and k
 *   (B,S,Hkv,D) with the step's cos / sin (B,S,D) bf16, and v (B,S,Hkv,D)
 *   copied alongside (v and v_out may be NULL), so the three outputs can
 *   share one buffer and its strides.  Every tensor has element strides
 *   (batch, seq, head) and a contiguous head_dim; D a multiple of 16.
 * wgkv_rope_qkv_norm -- wgkv_rope_qkv after Qwen3's per-head q_norm / k_norm
 *   (src/modeling_qwen3.py:235-239; weights of head_dim bf16, either may be
 *   NULL): x = bf16(w * bf16(x * rsqrt(mean_head(x^2) + eps))) before the
 *   rotation; k_pre (may be NULL; needs k_norm_weight) receives the
 *   normalised, unrotated k (the gate's pre-RoPE key) with strides (batch,
 *   seq, head).  head_dim <= 256 with a norm.
 * wgkv_silu_mul -- LlamaMLP's act_fn(gate) * up (:161): rows of `cols`
 *   bf16 (cols a multiple of 8), gate and up with their own row strides
 *   (e.g. the two halves of one fused projection), out contiguous.
 * wgkv_gemv -- the one-row nn.Linear of a decode step (LlamaAttention's
 *   q/k/v and o projections, :252-323 of modeling_llama.py; LlamaMLP :149-161;
 *   the LM head): y = W x with W (n, k) bf16 (row stride w_row_stride), x
 *   (k) bf16, fp32 accumulation, y bf16 (k a multiple of 8, <= 32768; W and
 *   x 16-byte aligned).  mode 0: y = bf16(W x) (n values).  mode 1: y =
 *   bf16(residual + bf16(W x)), the residual add after the projection
 *   (residual (n) bf16; y may equal residual).  mode 2: W holds the gate
 *   rows 0..n-1 and the up rows n..2n-1 (one stacked [gate; up] weight) and
 *   y = bf16(bf16(silu(bf16(W_gate x))) * bf16(W_up x)) (n values).
 * wgkv_gemv_ex -- wgkv_gemv with two fusions of a decode step.  With
 *   norm_weight (k) the workgroups first apply wgkv_rms_norm to x (with
 *   norm_residual: to x + norm_residual, stored to norm_residual_out), bit
 *   for bit, and multiply the normalised row.  mode 3 is LlamaAttention's
 *   q/k/v projection with apply_rotary_pos_emb (modeling_llama.py:265-271):
 *   W holds the q, k and v rows of num_q_heads + 2 num_kv_heads heads of
 *   head_dim (n = that many rows); y (n) gets the rotated q and k (cos, sin:
 *   head_dim bf16 values of the token's position, wgkv_rope_qkv's rounding)
 *   and v, in W's row order; k_raw (num_kv_heads * head_dim) the unrotated
 *   k (the gate's pre-RoPE key).
 * ---------------------------------------------------------------------- */
int wgkv_rms_norm(const void* x, int64_t x_row_stride, const void* residual, int64_t res_row_stride,
                  const void* weight, void* out, int64_t out_row_stride, void* residual_out,
                  int64_t res_out_row_stride, int32_t rows, int32_t hidden, float eps, void* stream);

int wgkv_rope_qkv(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                  const void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                  const void* v, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                  const void* cos, const void* sin, int64_t cs_sb, int64_t cs_ss,
                  void* q_out, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                  void* k_out, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                  void* v_out, int64_t vo_sb, int64_t vo_ss, int64_t vo_sh,
                  int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                  int32_t head_dim, void* stream);

int wgkv_rope_qkv_norm(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                       const void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                       const void* v, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                       const void* cos, const void* sin, int64_t cs_sb, int64_t cs_ss,
                       void* q_out, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                       void* k_out, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                       void* v_out, int64_t vo_sb, int64_t vo_ss, int64_t vo_sh,
                       int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t head_dim, const void* q_norm_weight, const void* k_norm_weight, float eps,
                       void* k_pre, int64_t kp_sb, int64_t kp_ss, int64_t kp_sh, void* stream);

int wgkv_silu_mul(const void* gate, int64_t gate_row_stride, const void* up, int64_t up_row_stride,
                  void* out, int64_t rows, int32_t cols, void* stream);

int wgkv_gemv(const void* w, int64_t w_row_stride, int32_t n, int32_t k, const void* x, void* y,
              int32_t mode, const void* residual, void* stream);

int wgkv_gemv_ex(const void* w, int64_t w_row_stride, int32_t n, int32_t k, const void* x, void* y,
                 int32_t mode, const void* residual,
                 const void* norm_weight, const void* norm_residual, void* norm_residual_out, float eps,
                 const void* cos, const void* sin, void* k_raw,
                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, void* stream);

/* wgkv_qkv_rope_ring_write -- wgkv_gemv_ex mode 3 (optional norm_weight
 * prologue; n = (num_q_heads + 2 num_kv_heads) * head_dim rows) whose
 * workgroups also do the decode step's ring write of a layer under deferred
 * gating, i.e. what wgkv_decode_append_ring does with no mask, no promotion
 * and no advance (decode_wrapper's write, src/modeling_layers.py:1390-1407,
 * and the attention lengths, :1429-1432): with (local_ptr, local_length) =
 * ring_state[0..1] and slot = local_length < W ? local_length : local_ptr,
 * the rotated k, v and the unrotated k of KV head h go to ring row
 * (layer, h, slot) of pool_k, pool_v (token rows of head_dim, the ring at
 * rows ((layer * num_kv_heads + h) * W + slot)) and local_pre_key
 * (num_layers, num_kv_heads, W, head_dim); cache_seqlens (the layer's
 * num_kv_heads values) = min(local_length + 1, W) + global_lengths[layer *
 * num_kv_heads + h]; ring_state[2] = slot.  The ring pointers are not
 * advanced.  A promotion that reads the slot (the first layer's) must run
 * before the call.  num_kv_heads <= 64.  No counterpart in the reference,
 * which writes the ring after its projections: one launch fewer per layer
 * for graph-captured decode steps. */
int wgkv_qkv_rope_ring_write(const void* w, int64_t w_row_stride, int32_t k, const void* x, void* y,
                             const void* norm_weight, float eps, const void* cos, const void* sin, void* k_raw,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t layer, int32_t num_layers, int32_t local_window, int32_t* ring_state,
                             void* pool_k, void* pool_v, void* local_pre_key,
                             const int32_t* global_lengths, int32_t* cache_seqlens, void* stream);

/* wgkv_rope_qkv_norm_ring_write -- wgkv_rope_qkv_norm for one decode row
 * (batch = seq_len = 1; element strides between heads only; v and v_out
 * required) whose threads also do the ring write of wgkv_qkv_rope_ring_write
 * (same ring arguments and layout): the rotated k, v and the pre-RoPE k --
 * after Qwen3's k head norm when k_norm_weight is given -- into ring row
 * (layer, h, slot), the layer's attention lengths and ring_state[2] = slot;
 * pool_k, pool_v and local_pre_key 16-byte aligned.  For decode steps whose
 * q/k head norms keep RoPE out of the q/k/v product's epilogue
 * (modeling_qwen3.py:235-239).  No counterpart in the reference, which
 * writes the ring after its projections (modeling_layers.py:1390-1407). */
int wgkv_rope_qkv_norm_ring_write(const void* q, int64_t q_sh, const void* k, int64_t k_sh,
                                  const void* v, int64_t v_sh, const void* cos, const void* sin,
                                  void* q_out, int64_t qo_sh, void* k_out, int64_t ko_sh,
                                  void* v_out, int64_t vo_sh,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  const void* q_norm_weight, const void* k_norm_weight, float eps,
                                  void* k_pre, int64_t kp_sh,
                                  int32_t layer, int32_t num_layers, int32_t local_window,
                                  int32_t* ring_state, void* pool_k, void* pool_v, void* local_pre_key,
                                  const int32_t* global_lengths, int32_t* cache_seqlens, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WGKV_H_ */
