/*
 * ukv.h - C ABI of libukv.so, the MI355X (gfx950) Page16 hot path of BP-KV.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * enqueues its kernels on the given HIP stream and returns without a host
 * synchronisation. Return value: UKV_OK (0) or a negative ukv_status.
 * No entry point allocates device memory: scratch space is passed in as a
 * workspace whose size the matching *_workspace_bytes() call reports.
 *
 * Reference interfaces replaced (paths relative to the BP-KV repository):
 *   ukv_page16_decode      core/page16_native.py:83-150 page16_decode_attention
 *                          (kernel core/page16_native.py:17-80)
 */
#ifndef UKV_H_
#define UKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ukv_stream_t; /* hipStream_t; NULL = default stream */

/* Element types of q / K / V / out (16-bit floating point only). */
#define UKV_DTYPE_F16 0
#define UKV_DTYPE_BF16 1

enum ukv_status {
  UKV_OK = 0,
  UKV_ERR_INVALID_ARGUMENT = -1, /* null pointer or negative size */
  UKV_ERR_EMPTY = -2,            /* batch, num_q_heads or head_dim <= 0 */
  UKV_ERR_GQA = -3,              /* n_rep < 1, or q heads map past num_kv_heads */
  UKV_ERR_HEAD_DIM = -4,         /* head_dim > 256 */
  UKV_ERR_DTYPE = -5,            /* dtype is not UKV_DTYPE_F16 / UKV_DTYPE_BF16 */
  UKV_ERR_WORKSPACE = -6,        /* workspace missing or smaller than required */
  UKV_ERR_LAUNCH = -7,           /* the HIP runtime rejected a kernel launch */
  UKV_ERR_NO_DEVICE = -8         /* no gfx950 device is current */
};

/* Library version, (major << 16) | (minor << 8) | patch. */
int ukv_version(void);

/* Static text for a ukv_status value. */
const char* ukv_status_string(int status);

/*
 * Bytes of workspace ukv_page16_decode needs for this shape. The workspace
 * holds the split-K partial results (never read before written), so it needs
 * no initialisation and may be reused by consecutive calls on one stream.
 */
size_t ukv_page16_workspace_bytes(int batch, int num_q_heads, int head_dim, int max_blocks);

/*
 * Page16 paged decode attention: one query token per sequence over 16-token
 * KV pages. Replaces core/page16_native.py:83-150 (page16_decode_attention)
 * and its Triton kernel core/page16_native.py:17-80.
 *
 *   q            [batch, num_q_heads, head_dim], element strides q_strides[0..1],
 *                last dimension contiguous
 *   k_cache      [num_pages, 16, num_kv_heads, head_dim] page/token/head element
 *   v_cache      strides k_strides[0..2] / v_strides[0..2], last dim contiguous
 *   block_table  int32 [batch, max_blocks], row-major; entry j of row b is the
 *                physical page holding tokens 16j..16j+15 of sequence b
 *   seqlens      int32 [batch], tokens to attend per sequence (including the
 *                current token); clamped to [0, 16*max_blocks]
 *   out          [batch, num_q_heads, head_dim] contiguous, same dtype as q
 *
 * q head h reads KV head h / n_rep. For each (b, h):
 *   out = sum_t softmax_t(softmax_scale * <q, K_t>) * V_t,  t < seqlens[b],
 * accumulated in fp32 and rounded to dtype. A sequence with no token yields
 * NaN (0/0), as in the reference. A block-table entry outside [0, num_pages)
 * is treated as a page whose tokens are all masked (the reference reads out of
 * bounds there), so the kernel never leaves the pool.
 */
int ukv_page16_decode(const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* block_table, const int32_t* seqlens, void* out,
                      int batch, int num_q_heads, int num_kv_heads, int head_dim, int n_rep,
                      int max_blocks, int num_pages, const int64_t* q_strides,
                      const int64_t* k_strides, const int64_t* v_strides, float softmax_scale,
                      int dtype, void* workspace, size_t workspace_bytes, ukv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* UKV_H_ */
