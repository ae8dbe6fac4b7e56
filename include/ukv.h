/*
 * ukv.h - C ABI of libukv.so, the MI355X (gfx950) Page16 hot path of BP-KV.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * enqueues its kernels on the given HIP stream and returns without a host
 * synchronisation. Return value: UKV_OK (0) or a negative ukv_status.
 * No entry point allocates device memory: scratch space is passed in as a
 * workspace whose size the matching *_workspace_bytes() call reports, except for
 * ukv_page16_decode_noalloc, whose scratch is a fixed device array of the library.
 *
 * Reference interfaces replaced (paths relative to the BP-KV repository):
 *   ukv_page16_decode      core/page16_native.py:83-150 page16_decode_attention
 *                          (kernel core/page16_native.py:17-80)
 *   ukv_kv_scatter_tokens  core/pool.py:127-141 PagedKVPool.write_kv_to_blocks
 *   ukv_kv_gather_tokens   core/pool.py:154-172 PagedKVPool.read_kv_from_blocks
 *   ukv_page_copy          core/scheduler.py:702-733 _write_block_indexed_layer_to_pool (page gather),
 *                          core/offload.py:1236-1262 prune_sequence_window (pool->pool compaction),
 *                          core/offload.py:163-179, 577-597, 662-680 per-page offload/prefetch copies
 *   ukv_kv_append          core/scheduler.py:401-408 decode-token scatter into the pool
 *   ukv_copy_2d            core/offload.py:577-597, 662-680 per-page pinned copies (one strided copy per chunk)
 *   ukv_page16_decode_append  core/scheduler.py:401-418 that scatter fused with the decode call
 *   ukv_retain_writeback_dense  core/scheduler.py:702-733, 735-799 selected writeback of dense raw KV
 *                          (block-indexed and token-granular), all layers of a sequence in one launch
 *   ukv_retain_compact_pages    the same map over pool-resident pages; core/offload.py:1236-1258
 *                          prune_sequence_window's pool->pool copy
 *   ukv_decode_prologue    core/offload.py:780-866 reserve_decode_slot (table side),
 *                          core/scheduler.py:1092-1160 per-layer table / cache_seqlens build,
 *                          core/scheduler.py:1247-1265 commit (seq_len += 1)
 *   ukv_select_topk        core/scheduler.py:613-616, core/compress.py:141-142 block top-k + sort
 *   ukv_snapkv_scores      core/scheduler.py:565-592 _score_layer_blocks_for_selection
 *                          (core/compress.py:116-130): observation-window block importance
 *   ukv_kv_write_varlen    core/pool.py:127-141 for a prefill chunk appended after its prefix
 *   ukv_paged_prefill      core/engine.py:1826-1854 chunked prefill attention over past KV
 *                          (HF attention / core/varlen.py:19-42 flash_attn_varlen_func, causal)
 *   ukv_paged_prefill_obs_stats  that attention, also producing the observation window's
 *                          softmax normalisers (core/scheduler.py:269-341 q-tail capture +
 *                          the first half of core/scheduler.py:565-592)
 *   ukv_snapkv_scores_from_stats  ukv_snapkv_scores taking those normalisers
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

/*
 * Asynchronous strided copy of `height` rows of `width` bytes between device memory and pinned
 * host memory (either direction, hipMemcpy2DAsync with the direction inferred), on `stream`.
 * The pinned page arena moves a chunk of pages of every layer with one call (one row per layer).
 * Replaces the per-(layer, page) pinned allocations and small copies of core/offload.py:577-597
 * (offload) and 662-680 (prefetch).
 */
int ukv_copy_2d(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width, size_t height,
                ukv_stream_t stream);

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

/*
 * ukv_page16_decode without a workspace argument: the split-K scratch is a device array of
 * the library (UKV_PAGE16_SCRATCH_BYTES per GPU, held by each GPU the library runs on until
 * the process ends), so the call allocates nothing - no hipMalloc, hipFree or allocating
 * library routine. Same arguments (less the workspace), semantics and result as
 * ukv_page16_decode; UKV_ERR_WORKSPACE (nothing launched) when the shape needs more than
 * UKV_PAGE16_SCRATCH_BYTES (ukv_page16_workspace_bytes), UKV_ERR_NO_DEVICE when the array's
 * address cannot be read on the current device. Every call on one GPU uses that GPU's one
 * array: calls that overlap there (two streams, two host threads) race.
 * No counterpart in the reference: this is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 */
#define UKV_PAGE16_SCRATCH_BYTES ((size_t)32 << 20)
int ukv_page16_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_table, const int32_t* seqlens, void* out,
                              int batch, int num_q_heads, int num_kv_heads, int head_dim, int n_rep,
                              int max_blocks, int num_pages, const int64_t* q_strides,
                              const int64_t* k_strides, const int64_t* v_strides, float softmax_scale,
                              int dtype, ukv_stream_t stream);

/*
 * Decode with the step's token append fused in: the same result as ukv_kv_append with
 * old_lens = seqlens - 1 (block_size 16) followed by ukv_page16_decode over seqlens, in one
 * call. k_new / v_new are [batch, num_kv_heads, head_dim] rows with element strides
 * new_strides[0..1] = {batch, head}; the token of sequence b is written to position
 * seqlens[b] - 1 unless seqlens[b] <= 0, the position is beyond max_blocks * 16 or its page
 * id is outside [0, num_pages). The split kernel writes the rows itself while it reads that
 * page (one launch fewer per layer); shapes it does not take run the append kernel first.
 * Precondition of the fused form: no page that one sequence attends is the page another
 * sequence's token is written to. The pool gives every sequence pages of its own, so this
 * holds unless a length exceeds its table row (then its zero padding, page 0, is attended;
 * the reference's index_put rejects such a length). Where it fails, that page's read races
 * with the write: call ukv_kv_append, then ukv_page16_decode.
 * Workspace as for ukv_page16_decode. Replaces core/scheduler.py:401-418 (block_pos / tok_pos,
 * the K and V index_put, attn_lens = old_lens + 1, page16_decode_attention).
 */
int ukv_page16_decode_append(const void* q, void* k_cache, void* v_cache, const int32_t* block_table,
                             const int32_t* seqlens, const void* k_new, const void* v_new,
                             const int64_t* new_strides, void* out, int batch, int num_q_heads,
                             int num_kv_heads, int head_dim, int n_rep, int max_blocks, int num_pages,
                             const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                             float softmax_scale, int dtype, void* workspace, size_t workspace_bytes,
                             ukv_stream_t stream);

/*
 * Token rows <-> pages for one layer of the pool (bit-exact copies).
 *   pool_layer   [num_pages, block_size, num_heads, head_dim], element strides pool_strides[0..2]
 *                (page, token, head); last dimension contiguous
 *   dense        [num_heads, n_tokens, head_dim], element strides dense_strides[0..1]
 *                (head, token); last dimension contiguous (the reference's [H_kv, T, D])
 *   page_ids     int32 [n_ids] device array; token t lives in page page_ids[t / block_size],
 *                slot t % block_size
 * Requires n_tokens <= block_size * n_ids. Page ids outside [0, num_pages) are skipped.
 * Replace core/pool.py:127-141 (write_kv_to_blocks) and :154-172 (read_kv_from_blocks).
 */
int ukv_kv_scatter_tokens(void* pool_layer, const int64_t* pool_strides, const void* dense,
                          const int64_t* dense_strides, const int32_t* page_ids, int n_ids, int num_pages,
                          int n_tokens, int block_size, int num_heads, int head_dim, ukv_stream_t stream);
int ukv_kv_gather_tokens(const void* pool_layer, const int64_t* pool_strides, void* dense,
                         const int64_t* dense_strides, const int32_t* page_ids, int n_ids, int num_pages,
                         int n_tokens, int block_size, int num_heads, int head_dim, ukv_stream_t stream);

/*
 * Whole-page copies across layers, for npools (1 or 2: K and V) pool pairs:
 *   dst_pools[p][layer, dst_ids[layer*dst_ids_layer_stride + j]] =
 *       src_pools[p][layer, src_ids[layer*src_ids_layer_stride + j]]      j < n, layer < layers
 * A pool is [layers, pages, page_elems] with element strides {layer, page} given in
 * src_strides / dst_strides; a page is page_elems contiguous 16-bit elements (multiple of 8).
 * An id list stride of 0 shares one list across layers. Ids outside [0, src_pages) /
 * [0, dst_pages) skip that copy. Destination pages must not be source pages of the same call.
 * Replaces the per-layer index_select / index_put of core/scheduler.py:702-733, the pool->pool
 * copy of core/offload.py:1236-1262, and the per-page copies of core/offload.py:577-597, 662-680.
 */
int ukv_page_copy(const void* const* src_pools, void* const* dst_pools, int npools, const int64_t* src_strides,
                  const int64_t* dst_strides, const int32_t* src_ids, int64_t src_ids_layer_stride,
                  const int32_t* dst_ids, int64_t dst_ids_layer_stride, int n, int layers, int page_elems,
                  int src_pages, int dst_pages, ukv_stream_t stream);

/*
 * Retain-set writeback: one launch writes the retained tokens of every layer of one sequence into
 * its destination pages (dst_ids, shared by every layer; [layers, num_pages, 16, num_heads,
 * head_dim] K/V pools with element strides pool_strides = {layer, page, slot, head}). Destination
 * position p < dst_len of layer l takes source token
 *   p                                          if p < sink_len;
 *   sink_len + 16*sel[l*sel_layer_stride + j] + r,  j = (p - sink_len)/16, r = (p - sink_len)%16,
 *                                              if p < sink_len + 16*k; when that token is not below
 *                                              mid_end = max(sink_len, src_len - obs_len) (or the
 *                                              entry is negative) the row is zero if pad_blocks,
 *                                              else not written;
 *   obs_start + (p - sink_len - 16*k)          otherwise, obs_start = max(0, src_len - obs_len);
 * dst_len = sink_len + 16*k + (src_len - obs_start), and position p goes to page dst_ids[p/16],
 * slot p%16 (slots past dst_len are not written). This is the SnapKV compaction layout - the sink,
 * each selected middle block zero-padded to 16 tokens, the observation window - at any alignment.
 * Requires sink_len <= src_len, dst_len <= 16*n_dst_ids, head_dim % 8 == 0 and 16-byte aligned
 * rows, else UKV_ERR_INVALID_ARGUMENT; destination ids outside [0, num_pages) skip their page.
 *
 * ukv_retain_writeback_dense: sources are the scheduler's dense raw K/V of each layer,
 * k_layers[l] / v_layers[l] (HOST arrays of `layers` device pointers) [num_heads, src_len,
 * head_dim] with element strides dense_strides = {head, token}. Replaces the per-layer selected
 * writeback of core/scheduler.py:735-799 (_write_selected_layer_to_pool: the block-aligned fast
 * path's index_select -> permute().contiguous() -> index_put of _write_block_indexed_layer_to_pool
 * :702-733, with sink_len = obs_len = 0 and sel = the source blocks, and the token-granular
 * _write_piece_to_blocks :666-690 / _pad_piece_to_block :692-700 path) for all layers of a
 * sequence at once (core/scheduler.py:826-848).
 *
 * ukv_retain_compact_pages: sources are pool-resident pages, token t of layer l at page
 * src_ids[t/16], slot t%16 of k_src_pool / v_src_pool (strides src_strides = {layer, page, slot,
 * head}; ids outside [0, src_num_pages) skip the token); src_len <= 16*n_src_ids. Source and
 * destination pages must not overlap. With sink_len = obs_len = 0, pad_blocks = 0 and sel = the
 * kept blocks in ascending order, shared by all layers (sel_layer_stride 0), this is the
 * pool->pool copy of core/offload.py:1236-1258 (prune_sequence_window: each kept block's tokens,
 * a partial last block included, concatenated into new pages); with the SnapKV map it is the
 * selected writeback of a sequence whose KV is already in pages.
 */
int ukv_retain_writeback_dense(const void* const* k_layers, const void* const* v_layers, const int64_t* dense_strides,
                               int src_len, int sink_len, int obs_len, const int32_t* sel, int64_t sel_layer_stride,
                               int k, int pad_blocks, void* k_pool, void* v_pool, const int64_t* pool_strides,
                               const int32_t* dst_ids, int n_dst_ids, int num_pages, int layers, int num_heads,
                               int head_dim, ukv_stream_t stream);
int ukv_retain_compact_pages(const void* k_src_pool, const void* v_src_pool, const int64_t* src_strides,
                             const int32_t* src_ids, int n_src_ids, int src_num_pages, int src_len, int sink_len,
                             int obs_len, const int32_t* sel, int64_t sel_layer_stride, int k, int pad_blocks,
                             void* k_pool, void* v_pool, const int64_t* pool_strides, const int32_t* dst_ids,
                             int n_dst_ids, int num_pages, int layers, int num_heads, int head_dim,
                             ukv_stream_t stream);

/*
 * Decode-step append: for each sequence b with len = old_lens[b], write k_new[b] / v_new[b]
 * ([num_heads, head_dim] rows, strides new_strides[0..1] = {batch, head}) into page
 * block_table[b, len / block_size], slot len % block_size of the layer's K / V pool, and, if new_lens is not
 * NULL, store len + 1. Sequences whose page index is >= max_blocks or whose page id is outside
 * [0, num_pages) are not written. Replaces core/scheduler.py:401-408.
 */
int ukv_kv_append(void* k_pool_layer, void* v_pool_layer, const int64_t* k_strides, const int64_t* v_strides,
                  const void* k_new, const void* v_new, const int64_t* new_strides, const int32_t* block_table,
                  int max_blocks, const int32_t* old_lens, int32_t* new_lens, int batch, int block_size,
                  int num_heads, int head_dim, int num_pages, ukv_stream_t stream);

/*
 * Once per decode step, shared by every layer (the table and lengths are the same for all
 * layers): writes the step's new pages into the device block table and the attention
 * lengths. new_pages is a HOST array of n_new (row, col, page id) int32 triples; each sets
 * block_table[row * max_blocks + col] = page id. Every row must be in [0, batch) and every
 * col in [0, max_blocks), else UKV_ERR_INVALID_ARGUMENT and nothing is launched. If lens_out
 * is not NULL, lens_out[b] = lens_in[b] + 1 for b < batch (lens_out may equal lens_in). The
 * triples travel as kernel arguments (no host-to-device copy; one launch per 128 triples).
 * Replaces the table side of core/offload.py:780-866 (reserve_decode_slot: the new block
 * id appended to every layer's gpu_block_map), the per-layer build_block_table and
 * cache_seqlens of core/scheduler.py:1092-1160, and the seq_len += 1 loop of
 * core/scheduler.py:1247-1265.
 */
int ukv_decode_prologue(int32_t* block_table, int max_blocks, int batch, const int32_t* lens_in,
                        int32_t* lens_out, const int32_t* new_pages, int n_new, ukv_stream_t stream);

/*
 * Retain-set selection: for each row r, the k_r indices i < n_r with the largest scores
 * (float32 scores[r * row_stride + i]), ties (-0 and +0 are equal) to the lower index, NaN
 * ranked above every number, written to out[r * out_stride + 0 .. k_r-1] in ascending order;
 * the remaining entries up to k_max are set to -1. row_n / row_k are optional int32 [rows] device arrays
 * (NULL: n_max / k_max for every row); k_r is clamped to [0, min(n_r, k_max)].
 * Replaces torch.topk + sort of core/scheduler.py:613-616 and core/compress.py:141-142, whose
 * order of equal scores is unspecified.
 */
int ukv_select_topk(const float* scores, int64_t row_stride, const int32_t* row_n, const int32_t* row_k, int rows,
                    int n_max, int k_max, int32_t* out, int64_t out_stride, ukv_stream_t stream);

/*
 * Prefill-chunk K/V into pages: for sequence b with chunk rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1
 * (C_b rows) and kv_lens[b] keys after the chunk, row cu_seqlens_q[b] + i of k_new / v_new
 * ([total, num_heads, head_dim], strides new_strides = {row, head}) goes to position
 * P_b + i = kv_lens[b] - C_b + i: page block_table[b, pos / 16], slot pos % 16. Positions outside
 * [0, 16*max_blocks) and page ids outside [0, num_pages) are skipped. max_chunk bounds C_b: rows
 * i >= max_chunk of a longer chunk are not written (ukv_paged_prefill with the same max_chunk then
 * returns NaN rows for that sequence).
 */
int ukv_kv_write_varlen(void* k_pool_layer, void* v_pool_layer, const int64_t* k_strides, const int64_t* v_strides,
                        const void* k_new, const void* v_new, const int64_t* new_strides, const int32_t* block_table,
                        int max_blocks, const int32_t* cu_seqlens_q, const int32_t* kv_lens, int batch,
                        int max_chunk, int num_heads, int head_dim, int num_pages, ukv_stream_t stream);

/*
 * Chunked prefill attention over the paged pool. Query row cu_seqlens_q[b] + i (i < C_b) of
 * sequence b is at position P_b + i, P_b = kv_lens[b] - C_b, and attends to keys
 * 0 .. P_b + i of the sequence (causal, bottom-right aligned) read through block_table
 * ([batch, max_blocks] int32, 16-token pages, keys already written - see ukv_kv_write_varlen);
 * q head h reads KV head h / n_rep.
 *   q    [total_q, num_q_heads, head_dim], element strides q_strides = {row, head}
 *   k/v  [num_pages, 16, num_kv_heads, head_dim], strides {page, token, head}
 *   out  [total_q, num_q_heads, head_dim] contiguous, q's dtype
 * fp32 softmax and accumulation; a row with no visible key yields NaN. max_chunk bounds C_b (the
 * flash-attn max_seqlen_q, core/varlen.py:28-29, which the Python wrapper derives from or checks
 * against host lengths): the block plan covers max_chunk queries per sequence, and every row of a
 * sequence whose C_b exceeds it is written as NaN (its chunk K/V were not all written either), so an
 * understated max_chunk on device-only lengths is loud, never stale memory. max_chunk * batch
 * below total_q (necessarily understated) is UKV_ERR_INVALID_ARGUMENT before any launch.
 * Replaces the dense chunked prefill of core/engine.py:1826-1854 (HF attention over the past
 * KV) and core/varlen.py:19-42 (flash_attn_varlen_func, causal=True).
 */
int ukv_paged_prefill(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                      const int32_t* cu_seqlens_q, const int32_t* kv_lens, void* out, int batch, int total_q,
                      int max_chunk, int num_q_heads, int num_kv_heads, int head_dim, int n_rep, int max_blocks,
                      int num_pages, const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                      float softmax_scale, int dtype, ukv_stream_t stream);

/*
 * ukv_paged_prefill, and for the chunk's last obs_len queries of every sequence also SnapKV's
 * row statistics over that sequence's middle keys (what ukv_snapkv_scores' first pass computes
 * when the chunk is the sequence's last, L = kv_lens[b]): for q head h and window query i
 * (chunk row C_b - obs_len + i),
 *   obs_stats[2 * (b * stats_seq_stride + h * obs_len + i)]     = log2 of the sum over keys
 *       j in [sink_len, L - obs_len), and the zero rows padding them to a multiple of 16, of
 *       2^(q.k_j * softmax_scale * log2(e)) (a zero row scores 0);
 *   obs_stats[2 * (b * stats_seq_stride + h * obs_len + i) + 1] = 0, or 1 where that sum fell
 *       below 2^-100 of the query's largest weight, or where the sink and window keys hold half of
 *       the query's weight or more (its low bits are lost; ukv_snapkv_scores_from_stats recomputes
 *       such items).
 * stats_seq_stride counts (value, flag) pairs and is at least num_q_heads * obs_len; obs_stats is
 * 8-byte aligned. For the layout ukv_snapkv_scores_from_stats reads ([seqs][layers][num_q_heads]
 * [obs_len] pairs) pass obs_stats + 2 * layer * num_q_heads * obs_len and stats_seq_stride =
 * layers * num_q_heads * obs_len. The rows come from the tiled kernel (head_dim 128, n_rep
 * 1/2/4/8/16, 16-byte aligned rows); on the scalar path every row is written flagged (0, 1), so the
 * scores recompute them. C_b >= obs_len for the rows to exist.
 * The reference captures the window's queries in its q_proj hook (core/scheduler.py:269-341)
 * and normalises their softmax over K_mid at selection time (core/scheduler.py:565-592,
 * core/compress.py:116-130); here that normaliser comes from the prefill's own softmax
 * denominators: the prefill kernel leaves each window row's running max and denominator (the sum
 * of its fp16-rounded weights over every key it sees) in obs_stats, and a second kernel on the
 * same stream sums the sink and window keys' weights again (fp32, from the same scores) and takes
 * them off. Relative error of the sum: that of fp16-rounded weights (2^-11 each, random sign), at
 * most doubled by the difference before the row is flagged.
 */
int ukv_paged_prefill_obs_stats(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                                const int32_t* cu_seqlens_q, const int32_t* kv_lens, void* out, int batch,
                                int total_q, int max_chunk, int num_q_heads, int num_kv_heads, int head_dim,
                                int n_rep, int max_blocks, int num_pages, const int64_t* q_strides,
                                const int64_t* k_strides, const int64_t* v_strides, float softmax_scale, int dtype,
                                int sink_len, int obs_len, float* obs_stats, int64_t stats_seq_stride,
                                ukv_stream_t stream);

/*
 * SnapKV observation-window block scores (the importance scores ukv_select_topk ranks).
 * For every item (layer l of sequence b, item = b * layers + l), with L = seq_len:
 *   K_mid = K[:, sink_len : L - obs_len, :] zero-padded to aligned = ceil(L_mid / block_size)
 *           * block_size keys;  A = softmax(Q_obs . repeat_kv(K_mid)^T * softmax_scale) over keys;
 *   s = A.mean(over the obs_len queries).max(over the num_q_heads heads);
 *   raw[n] = sum of s over keys [block_size * n, block_size * (n + 1));
 *   scores[item * scores_stride + n] = max(raw[n-1], raw[n], raw[n+1]) if N >= 3, else raw[n]
 * for n < N = ukv_snapkv_block_count(...), which is 0 (nothing written, UKV_OK) when
 * L < sink_len + obs_len + block_size. Scores, maxima and sums are fp32 from 16-bit inputs; each
 * softmax weight is rounded to fp16 (relative error <= 2^-11) where the matrix cores sum it.
 *   q_obs        [items, num_q_heads, obs_len, head_dim], element strides q_strides[0..2]
 *                {item, head, query}, last dimension contiguous
 *   k            K rows with element strides k_strides[0..3] = {layer, seq-or-page, token, head}:
 *                block_table NULL: token t of (b, l), head g at k + l*s0 + b*s1 + t*s2 + g*s3
 *                (dense [layers][seqs][L][H_kv][D] or any strided view);
 *                block_table [seqs, max_blocks] int32: page block_table[b][t / 16], slot t % 16 at
 *                k + l*s0 + page*s1 + slot*s2 + g*s3 (the pool [layers, N, 16, H_kv, D]); page ids
 *                outside [0, num_pages) read as zero rows
 * num_q_heads must equal num_kv_heads * n_rep (q head h reads KV head h / n_rep); block_size must
 * be 16 (the page size; the reference's SnapKV block); layers * seqs <= 65535; otherwise
 * UKV_ERR_INVALID_ARGUMENT. The workspace (ukv_snapkv_workspace_bytes) needs no initialisation.
 * Replaces core/scheduler.py:565-592 and the scoring steps of core/compress.py:116-130.
 */
int ukv_snapkv_block_count(int seq_len, int sink_len, int obs_len, int block_size);
size_t ukv_snapkv_workspace_bytes(int layers, int seqs, int seq_len, int sink_len, int obs_len, int num_q_heads,
                                  int num_kv_heads, int head_dim, int n_rep, int block_size);
int ukv_snapkv_scores(const void* q_obs, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                      const int32_t* block_table, int max_blocks, int num_pages, int layers, int seqs, int seq_len,
                      int sink_len, int obs_len, int num_q_heads, int num_kv_heads, int head_dim, int n_rep,
                      int block_size, float softmax_scale, int dtype, float* scores, int64_t scores_stride,
                      void* workspace, size_t workspace_bytes, ukv_stream_t stream);

/*
 * ukv_snapkv_scores with the row statistics given: obs_stats holds [items][num_q_heads][obs_len]
 * (value, flag) float pairs as ukv_paged_prefill_obs_stats writes them (8-byte aligned), so the
 * first pass over the keys runs only for items with a flagged or non-finite row. Same scores up
 * to the statistics' rounding; same arguments and workspace otherwise. Replaces, with
 * ukv_paged_prefill_obs_stats, the same steps as ukv_snapkv_scores (core/scheduler.py:565-592).
 */
int ukv_snapkv_scores_from_stats(const void* q_obs, const int64_t* q_strides, const void* k,
                                 const int64_t* k_strides, const int32_t* block_table, int max_blocks, int num_pages,
                                 int layers, int seqs, int seq_len, int sink_len, int obs_len, int num_q_heads,
                                 int num_kv_heads, int head_dim, int n_rep, int block_size, float softmax_scale,
                                 int dtype, const float* obs_stats, float* scores, int64_t scores_stride,
                                 void* workspace, size_t workspace_bytes, ukv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* UKV_H_ */
