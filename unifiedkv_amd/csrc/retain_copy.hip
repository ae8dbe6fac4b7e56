// Retain-set writeback into pages (gfx950): the token-granular copy behind SnapKV compaction.
//
// One map, taken from the reference's selected writeback, says which source token lands on each
// destination position p of a layer (pages of 16 tokens, block b = 16 tokens):
//   p <  sink                      source token p                          (the sink piece)
//   p <  sink + 16 k               j = (p - sink) / 16, r = (p - sink) % 16:
//                                  source token sink + 16 sel[layer][j] + r if it is below
//                                  mid_end = max(sink, src_len - obs); otherwise a zero row (pad)
//                                  or no write (no pad)                    (selected middle blocks)
//   p <  dst_len                   source token obs_start + (p - sink - 16 k),
//                                  obs_start = max(0, src_len - obs)       (the window)
// dst_len = sink + 16 k + (src_len - obs_start). With pad this is core/scheduler.py:781-799
// (_write_piece_to_blocks :666-690 of the sink, each selected block zero-padded to 16 by
// _pad_piece_to_block :692-700, then the window); with sink = obs = 0 it is the block-indexed
// writeback of core/scheduler.py:702-733 (sel = the source blocks) and, without pad, the
// pool->pool prune copy of core/offload.py:1236-1258 (sel = the kept blocks, ascending, so that
// only the last one may be partial).
//
// Sources are either the dense per-layer [H, src_len, D] K/V of the scheduler's raw KV cache
// (one base pointer per layer, carried in the kernel arguments) or pool-resident pages read
// through the sequence's page list. Destination pages are shared by every layer. Each workgroup
// copies (up to 1 KiB of) one token row of one destination page of one layer of K or V; slots
// past dst_len are left untouched, as the reference leaves them.
#include <algorithm>

#include "ukv_common.h"

namespace ukv {

constexpr int kRetainLayersPerLaunch = 64;

struct RetainArgs {
  const uint16_t* src[2][kRetainLayersPerLaunch];  // dense: per-layer bases; paged: [kv][0] = pool
  int64_t s_head, s_tok;                           // dense element strides {head, token}
  int64_t s_layer, s_page, s_slot;                 // paged element strides (head stride in s_head)
  const int32_t* src_ids;                          // paged: page of source tokens 16i .. 16i+15
  int src_pages;                                   // paged: valid ids are [0, src_pages)
  int paged;
  int sink, k, obs_start, mid_end, dst_len, pad;
  const int32_t* sel;
  int64_t sel_lstride;                             // 0: one selection shared by every layer
  uint16_t* dst[2];
  int64_t d_layer, d_page, d_slot, d_head;
  const int32_t* dst_ids;
  int dst_pages;
  int layer0;                                      // first layer of this launch
  int H, D;
};

// grid (16 * destination pages, layers of this launch, 2 * slices): block (16 * page + slot, layer,
// 2 * slice + kv) copies chunks [slice * 64, slice * 64 + 64) of one slot (token row) of a page, its
// H * D / 8 16-byte chunks of K (kv 0) or V (kv 1), one per thread. The slot's source is the same for
// the whole block, so its map lookups are scalar loads; small blocks keep many loads in flight per CU
// (the whole-page copy ran 30 % faster in 2 KiB blocks than in 32 KiB ones).
constexpr int kRetainThreads = 64;
__global__ void __launch_bounds__(kRetainThreads) retain_copy_kernel(const RetainArgs a) {
  const int page = blockIdx.x >> 4;
  const int slot = blockIdx.x & 15;
  const int ll = blockIdx.y;
  const int layer = a.layer0 + ll;
  const int kv = blockIdx.z & 1;
  const int c = (blockIdx.z >> 1) * kRetainThreads + threadIdx.x;
  const int per_head = a.D >> 3;  // 16-byte chunks of a row
  const int p = 16 * page + slot;
  if (p >= a.dst_len) return;  // slots past dst_len are left untouched (whole block)
  const int did = a.dst_ids[page];
  if ((unsigned)did >= (unsigned)a.dst_pages) return;  // whole block
  // The source token of destination position p, or a zero row (pad), or no write (whole block).
  int64_t s;
  bool zero = false;
  if (p < a.sink) {
    s = p;
  } else if (p < a.sink + 16 * a.k) {
    const int j = (p - a.sink) >> 4;
    const int blk = a.sel[(int64_t)layer * a.sel_lstride + j];
    s = (int64_t)a.sink + 16 * (int64_t)blk + ((p - a.sink) & 15);
    if (blk < 0 || s >= a.mid_end) {
      if (!a.pad) return;
      zero = true;
    }
  } else {
    s = (int64_t)a.obs_start + (p - a.sink - 16 * a.k);
  }
  int64_t off = 0;
  if (!zero) {
    if (a.paged) {
      const int pid = a.src_ids[s >> 4];
      if ((unsigned)pid >= (unsigned)a.src_pages) return;
      off = (int64_t)layer * a.s_layer + (int64_t)pid * a.s_page + (s & 15) * a.s_slot;
    } else {
      off = s * a.s_tok;
    }
  }
  if (c >= a.H * per_head) return;
  const int h = c / per_head;
  const int e = 8 * (c - h * per_head);
  u32x4 r = {0u, 0u, 0u, 0u};
  if (!zero) {
    const uint16_t* src = a.paged ? a.src[kv][0] : a.src[kv][ll];
    r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + off + (int64_t)h * a.s_head + e));
  }
  uint16_t* dst = a.dst[kv] + (int64_t)layer * a.d_layer + (int64_t)did * a.d_page;
  __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(dst + (int64_t)slot * a.d_slot + (int64_t)h * a.d_head + e));
}

namespace {

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool mul8(int64_t x) { return (x & 7) == 0; }

// The map's scalars; UKV_ERR_INVALID_ARGUMENT when the destination list cannot hold dst_len.
int fill_map(RetainArgs& a, int src_len, int sink_len, int obs_len, const int32_t* sel, int64_t sel_lstride, int k,
             int pad_blocks, int n_dst_ids) {
  if (src_len < 0 || sink_len < 0 || obs_len < 0 || k < 0 || n_dst_ids < 0) return UKV_ERR_INVALID_ARGUMENT;
  if (sink_len > src_len || (k > 0 && !sel)) return UKV_ERR_INVALID_ARGUMENT;
  const int obs_start = std::max(0, src_len - obs_len);
  const int64_t dst_len = (int64_t)sink_len + 16 * (int64_t)k + (src_len - obs_start);
  if (dst_len > 16 * (int64_t)n_dst_ids || dst_len > (int64_t)1 << 30) return UKV_ERR_INVALID_ARGUMENT;
  a.sink = sink_len;
  a.k = k;
  a.obs_start = obs_start;
  a.mid_end = std::max(sink_len, src_len - obs_len);
  a.dst_len = (int)dst_len;
  a.pad = pad_blocks != 0;
  a.sel = sel;
  a.sel_lstride = sel_lstride;
  return UKV_OK;
}

int fill_dst(RetainArgs& a, void* k_pool, void* v_pool, const int64_t* pool_strides, const int32_t* dst_ids,
             int num_pages, int num_heads, int head_dim) {
  if (!k_pool || !v_pool || !pool_strides || num_heads <= 0 || head_dim <= 0 || num_pages < 0)
    return UKV_ERR_INVALID_ARGUMENT;
  if (head_dim % 8 != 0 || !al16(k_pool) || !al16(v_pool)) return UKV_ERR_INVALID_ARGUMENT;
  for (int i = 0; i < 4; ++i)
    if (!mul8(pool_strides[i])) return UKV_ERR_INVALID_ARGUMENT;
  a.dst[0] = static_cast<uint16_t*>(k_pool);
  a.dst[1] = static_cast<uint16_t*>(v_pool);
  a.d_layer = pool_strides[0];
  a.d_page = pool_strides[1];
  a.d_slot = pool_strides[2];
  a.d_head = pool_strides[3];
  a.dst_ids = dst_ids;
  a.dst_pages = num_pages;
  a.H = num_heads;
  a.D = head_dim;
  return UKV_OK;
}

int launch_retain(RetainArgs a, int layers, const void* const* k_layers, const void* const* v_layers,
                  ukv_stream_t stream) {
  const int pages = (a.dst_len + 15) / 16;
  if (pages == 0 || layers == 0) return UKV_OK;
  const int slices = (a.H * (a.D / 8) + kRetainThreads - 1) / kRetainThreads;  // per slot
  if (2 * slices > 65535) return UKV_ERR_INVALID_ARGUMENT;
  if (!a.dst_ids) return UKV_ERR_INVALID_ARGUMENT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Every layer's dense K/V pointer is checked before the first launch: a refusal writes nothing.
  if (!a.paged)
    for (int i = 0; i < layers; ++i)
      if (!k_layers[i] || !v_layers[i] || !al16(k_layers[i]) || !al16(v_layers[i])) return UKV_ERR_INVALID_ARGUMENT;
  const int per = a.paged ? 65535 : kRetainLayersPerLaunch;
  for (int l0 = 0; l0 < layers; l0 += per) {
    RetainArgs b = a;
    const int nl = std::min(per, layers - l0);
    b.layer0 = l0;
    if (!a.paged) {
      for (int i = 0; i < nl; ++i) {
        b.src[0][i] = static_cast<const uint16_t*>(k_layers[l0 + i]);
        b.src[1][i] = static_cast<const uint16_t*>(v_layers[l0 + i]);
      }
    }
    hipLaunchKernelGGL(retain_copy_kernel, dim3(16 * pages, nl, 2 * slices), dim3(kRetainThreads), 0, s, b);
    if (hipGetLastError() != hipSuccess) return UKV_ERR_LAUNCH;
  }
  return UKV_OK;
}

}  // namespace
}  // namespace ukv

using namespace ukv;

extern "C" int ukv_retain_writeback_dense(const void* const* k_layers, const void* const* v_layers,
                                          const int64_t* dense_strides, int src_len, int sink_len, int obs_len,
                                          const int32_t* sel, int64_t sel_layer_stride, int k, int pad_blocks,
                                          void* k_pool, void* v_pool, const int64_t* pool_strides,
                                          const int32_t* dst_ids, int n_dst_ids, int num_pages, int layers,
                                          int num_heads, int head_dim, ukv_stream_t stream) {
  if (layers < 0 || !k_layers || !v_layers || !dense_strides) return UKV_ERR_INVALID_ARGUMENT;
  RetainArgs a{};
  int rc = fill_map(a, src_len, sink_len, obs_len, sel, sel_layer_stride, k, pad_blocks, n_dst_ids);
  if (rc != UKV_OK) return rc;
  rc = fill_dst(a, k_pool, v_pool, pool_strides, dst_ids, num_pages, num_heads, head_dim);
  if (rc != UKV_OK) return rc;
  if (!mul8(dense_strides[0]) || !mul8(dense_strides[1])) return UKV_ERR_INVALID_ARGUMENT;
  a.paged = 0;
  a.s_head = dense_strides[0];
  a.s_tok = dense_strides[1];
  return launch_retain(a, layers, k_layers, v_layers, stream);
}

extern "C" int ukv_retain_compact_pages(const void* k_src_pool, const void* v_src_pool, const int64_t* src_strides,
                                        const int32_t* src_ids, int n_src_ids, int src_num_pages, int src_len,
                                        int sink_len, int obs_len, const int32_t* sel, int64_t sel_layer_stride,
                                        int k, int pad_blocks, void* k_pool, void* v_pool,
                                        const int64_t* pool_strides, const int32_t* dst_ids, int n_dst_ids,
                                        int num_pages, int layers, int num_heads, int head_dim,
                                        ukv_stream_t stream) {
  if (layers < 0 || !k_src_pool || !v_src_pool || !src_strides || n_src_ids < 0 || src_num_pages < 0)
    return UKV_ERR_INVALID_ARGUMENT;
  if ((int64_t)src_len > 16 * (int64_t)n_src_ids || (src_len > 0 && !src_ids)) return UKV_ERR_INVALID_ARGUMENT;
  RetainArgs a{};
  int rc = fill_map(a, src_len, sink_len, obs_len, sel, sel_layer_stride, k, pad_blocks, n_dst_ids);
  if (rc != UKV_OK) return rc;
  rc = fill_dst(a, k_pool, v_pool, pool_strides, dst_ids, num_pages, num_heads, head_dim);
  if (rc != UKV_OK) return rc;
  for (int i = 0; i < 4; ++i)
    if (!mul8(src_strides[i])) return UKV_ERR_INVALID_ARGUMENT;
  if (!al16(k_src_pool) || !al16(v_src_pool)) return UKV_ERR_INVALID_ARGUMENT;
  a.paged = 1;
  a.src[0][0] = static_cast<const uint16_t*>(k_src_pool);
  a.src[1][0] = static_cast<const uint16_t*>(v_src_pool);
  a.s_layer = src_strides[0];
  a.s_page = src_strides[1];
  a.s_slot = src_strides[2];
  a.s_head = src_strides[3];
  a.src_ids = src_ids;
  a.src_pages = src_num_pages;
  if (layers > 65535) return UKV_ERR_INVALID_ARGUMENT;
  return launch_retain(a, layers, nullptr, nullptr, stream);
}
