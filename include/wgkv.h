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
 * {16,32,64}, G = Hq/Hkv in {1,2,4}, B*Hkv <= 2048.  Split planning happens
 * on the device; out-of-range lengths are clamped to max_pages*page_size and
 * out-of-range page ids to the pool, so no access leaves the buffers.
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

#ifdef __cplusplus
}
#endif

#endif /* WGKV_H_ */
