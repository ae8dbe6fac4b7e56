// Bit-exact page movement on the paged KV pool (gfx950).
//
//   ukv_kv_scatter_tokens  dense [H, T, D] -> pages            (core/pool.py:127-141)
//   ukv_kv_gather_tokens   pages -> dense [H, T, D]            (core/pool.py:154-172)
//   ukv_page_copy          whole pages, per layer, src ids per layer or shared, dst ids shared or per
//                          layer; compaction, pool->pool pruning and staging pack/unpack
//                          (core/scheduler.py:702-733, core/offload.py:1236-1262, 577-597, 662-680)
//   ukv_kv_append          the decode step's new K/V token into page bt[b, len/bs], slot len%bs
//                          (core/scheduler.py:401-408)
//   ukv_decode_prologue    once per decode step: the step's new page ids into the block table and
//                          the attention lengths lens + 1 (core/offload.py:780-866,
//                          core/scheduler.py:1092-1160, 1247-1265)
//
// All of them are HBM-bound copies of 16-byte chunks; every byte is read once and written once.
// Rows must be 16-byte aligned (D % 8 == 0 and aligned strides); a 2-byte element path covers
// other rows. Page ids outside [0, num_pages) are skipped, never dereferenced.
#include <algorithm>

#include "ukv_common.h"

namespace ukv {

struct TokenCopyArgs {
  uint16_t* pool;          // one layer: [N][16][H][D]
  int64_t p_sp, p_st, p_sh;
  uint16_t* dense;         // [H][T][D]
  int64_t d_sh, d_st;
  const int32_t* page_ids; // page of tokens bs*i .. bs*i+bs-1
  int n_ids, num_pages;
  int T, H, D, bs;
};

// One thread per 16-byte chunk; consecutive threads walk a token's heads and
// dims, so pool-side addresses are contiguous within a page row.
template <bool SCATTER, bool VEC>
__global__ void __launch_bounds__(256) token_copy_kernel(const TokenCopyArgs a) {
  const int per = VEC ? a.D / 8 : a.D;  // items per (token, head) row
  const int64_t total = (int64_t)a.T * a.H * per;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int c = (int)(idx % per);
    const int64_t rest = idx / per;
    const int h = (int)(rest % a.H);
    const int t = (int)(rest / a.H);
    const int page = a.page_ids[t / a.bs];
    if ((unsigned)page >= (unsigned)a.num_pages) continue;
    const int64_t e = VEC ? 8 * c : c;
    uint16_t* pp = a.pool + (int64_t)page * a.p_sp + (int64_t)(t % a.bs) * a.p_st + (int64_t)h * a.p_sh + e;
    uint16_t* dp = a.dense + (int64_t)h * a.d_sh + (int64_t)t * a.d_st + e;
    if (VEC) {
      if (SCATTER)
        *reinterpret_cast<u32x4*>(pp) = *reinterpret_cast<const u32x4*>(dp);
      else
        *reinterpret_cast<u32x4*>(dp) = *reinterpret_cast<const u32x4*>(pp);
    } else {
      if (SCATTER)
        *pp = *dp;
      else
        *dp = *pp;
    }
  }
}

// 16-byte path: block t copies token t's H * D / 8 chunks (thread it = (head, chunk)); the page
// lookup is one scalar load per block, the indices 32-bit. One 32K-token layer (H=8, D=128):
// 20.9 us scatter / 20.8 us gather (6.4 TB/s read + write), against 21.3 / 21.4 us for the
// grid-stride form below, which now serves unaligned rows only.
constexpr int kTokenThreads = 128;
template <bool SCATTER>
__global__ void __launch_bounds__(kTokenThreads) token_copy_vec_kernel(const TokenCopyArgs a) {
  const int t = blockIdx.x;
  const int page = a.page_ids[t / a.bs];
  if ((unsigned)page >= (unsigned)a.num_pages) return;
  const int per = a.D >> 3;
  uint16_t* prow = a.pool + (int64_t)page * a.p_sp + (int64_t)(t % a.bs) * a.p_st;
  uint16_t* drow = a.dense + (int64_t)t * a.d_st;
  for (int it = threadIdx.x; it < a.H * per; it += kTokenThreads) {
    const int h = it / per;
    const int e = 8 * (it - h * per);
    uint16_t* pp = prow + (int64_t)h * a.p_sh + e;
    uint16_t* dp = drow + (int64_t)h * a.d_sh + e;
    if (SCATTER)
      *reinterpret_cast<u32x4*>(pp) = *reinterpret_cast<const u32x4*>(dp);
    else
      *reinterpret_cast<u32x4*>(dp) = *reinterpret_cast<const u32x4*>(pp);
  }
}

struct PageCopyArgs {
  const uint16_t* src[2];
  uint16_t* dst[2];
  int64_t s_layer, s_page;  // element strides of the source pools
  int64_t d_layer, d_page;  // element strides of the destination pools
  const int32_t* src_ids;
  const int32_t* dst_ids;
  int64_t src_ids_lstride;  // 0: one id list shared by every layer
  int64_t dst_ids_lstride;
  int n, layers, npools, page_elems, src_pages, dst_pages;
};

// grid (page slices, n, layers * npools); each block of kCopyThreads threads
// copies one 16-byte chunk per thread (2 KiB) of one page, with a non-temporal
// store (the destination is not read back soon). Small blocks measured fastest
// for config 5a's 14 GB gather: 2 KiB blocks 6.21 TB/s read + write, 4 KiB
// blocks 6.15 (1 KiB the same), 4 KiB in two chunks per thread 5.99 (5.66 with
// ordinary stores), a whole 32 KiB page per block 4.07.
constexpr int kCopyThreads = 128;
__global__ void __launch_bounds__(kCopyThreads) page_copy_kernel(const PageCopyArgs a) {
  constexpr int kPer = 1;  // 16-byte chunks per thread per block-slice
  const int j = blockIdx.y;
  const int layer = blockIdx.z / a.npools;
  const int pool = blockIdx.z % a.npools;
  const int sid = a.src_ids[(int64_t)layer * a.src_ids_lstride + j];
  const int did = a.dst_ids[(int64_t)layer * a.dst_ids_lstride + j];
  if ((unsigned)sid >= (unsigned)a.src_pages || (unsigned)did >= (unsigned)a.dst_pages) return;
  const u32x4* s = reinterpret_cast<const u32x4*>(a.src[pool] + (int64_t)layer * a.s_layer + (int64_t)sid * a.s_page);
  u32x4* d = reinterpret_cast<u32x4*>(a.dst[pool] + (int64_t)layer * a.d_layer + (int64_t)did * a.d_page);
  const int chunks = a.page_elems / 8;
  const int base = blockIdx.x * (kCopyThreads * kPer) + threadIdx.x;
  u32x4 r[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = base + i * kCopyThreads;
    if (c < chunks) r[i] = __builtin_nontemporal_load(s + c);
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = base + i * kCopyThreads;
    if (c < chunks) __builtin_nontemporal_store(r[i], d + c);
  }
}

struct AppendArgs {
  uint16_t* k_pool;
  uint16_t* v_pool;
  int64_t k_sp, k_st, k_sh, v_sp, v_st, v_sh;
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t n_sb, n_sh;  // [B][H][D] strides of k_new / v_new
  const int32_t* block_table;
  int max_blocks;
  const int32_t* old_lens;
  int pos_offset;     // the token of sequence b goes to position old_lens[b] + pos_offset
  int32_t* new_lens;  // nullable: old_lens + 1
  int B, H, D, num_pages, bs;
  int vec;  // rows 16-byte aligned: copy 16-byte chunks
};

// grid (B); the block writes one token row of every head of sequence b.
__global__ void __launch_bounds__(256) kv_append_kernel(const AppendArgs a) {
  const int b = blockIdx.x;
  const int lv = a.old_lens[b];
  if (threadIdx.x == 0 && a.new_lens) a.new_lens[b] = lv + 1;
  const int len = lv + a.pos_offset;
  if (len < 0) return;
  const int blk = len / a.bs;
  if (blk >= a.max_blocks) return;
  const int page = a.block_table[(int64_t)b * a.max_blocks + blk];
  if ((unsigned)page >= (unsigned)a.num_pages) return;
  const int slot = len % a.bs;
  const bool vec = a.vec != 0;
  const int per = vec ? a.D / 8 : a.D;
  for (int i = threadIdx.x; i < a.H * per; i += blockDim.x) {
    const int h = i / per, c = i % per;
    const int64_t e = vec ? 8 * c : c;
    const int64_t src = (int64_t)b * a.n_sb + (int64_t)h * a.n_sh + e;
    uint16_t* kd = a.k_pool + (int64_t)page * a.k_sp + (int64_t)slot * a.k_st + (int64_t)h * a.k_sh + e;
    uint16_t* vd = a.v_pool + (int64_t)page * a.v_sp + (int64_t)slot * a.v_st + (int64_t)h * a.v_sh + e;
    if (vec) {
      *reinterpret_cast<u32x4*>(kd) = *reinterpret_cast<const u32x4*>(a.k_new + src);
      *reinterpret_cast<u32x4*>(vd) = *reinterpret_cast<const u32x4*>(a.v_new + src);
    } else {
      *kd = a.k_new[src];
      *vd = a.v_new[src];
    }
  }
}

// Kernel arguments carry up to kPrologueMax (row, col, page id) triples, so a
// decode step's new pages reach the table without a host-to-device copy.
constexpr int kPrologueMax = 128;

struct PrologueArgs {
  int32_t* bt;
  int max_blocks;
  int B;
  const int32_t* lens_in;
  int32_t* lens_out;  // nullable
  int n;
  int32_t trip[3 * kPrologueMax];
};

// One block: threads write the new table entries, then every sequence's
// attention length. lens_in may alias lens_out (each thread reads, then writes,
// its own element).
__global__ void __launch_bounds__(256) decode_prologue_kernel(const PrologueArgs a) {
  const int t = threadIdx.x;
  if (t < a.n) a.bt[(int64_t)a.trip[3 * t] * a.max_blocks + a.trip[3 * t + 1]] = a.trip[3 * t + 2];
  if (a.lens_out)
    for (int b = t; b < a.B; b += blockDim.x) a.lens_out[b] = a.lens_in[b] + 1;
}

namespace {

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool m8(int64_t x) { return (x & 7) == 0; }

int launch_token_copy(bool scatter, const TokenCopyArgs& a, hipStream_t stream) {
  const bool vec = (a.D % 8 == 0) && a16(a.pool) && a16(a.dense) && m8(a.p_sp) && m8(a.p_st) && m8(a.p_sh) &&
                   m8(a.d_sh) && m8(a.d_st);
  const int64_t per = vec ? a.D / 8 : a.D;
  const int64_t total = (int64_t)a.T * a.H * per;
  if (total == 0) return UKV_OK;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
  if (vec && scatter)
    hipLaunchKernelGGL((token_copy_vec_kernel<true>), dim3(a.T), dim3(kTokenThreads), 0, stream, a);
  else if (vec)
    hipLaunchKernelGGL((token_copy_vec_kernel<false>), dim3(a.T), dim3(kTokenThreads), 0, stream, a);
  else if (scatter)
    hipLaunchKernelGGL((token_copy_kernel<true, false>), dim3(blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((token_copy_kernel<false, false>), dim3(blocks), dim3(256), 0, stream, a);
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}

int token_copy(bool scatter, void* pool, const int64_t* pool_strides, void* dense, const int64_t* dense_strides,
               const int32_t* page_ids, int n_ids, int num_pages, int n_tokens, int block_size, int num_heads,
               int head_dim, ukv_stream_t stream) {
  if (n_tokens < 0 || n_ids < 0 || num_heads <= 0 || head_dim <= 0 || block_size <= 0)
    return UKV_ERR_INVALID_ARGUMENT;
  if ((int64_t)n_tokens > (int64_t)block_size * n_ids) return UKV_ERR_INVALID_ARGUMENT;
  if (n_tokens == 0) return UKV_OK;
  if (!pool || !dense || !page_ids || !pool_strides || !dense_strides) return UKV_ERR_INVALID_ARGUMENT;
  TokenCopyArgs a{};
  a.pool = static_cast<uint16_t*>(pool);
  a.p_sp = pool_strides[0];
  a.p_st = pool_strides[1];
  a.p_sh = pool_strides[2];
  a.dense = static_cast<uint16_t*>(dense);
  a.d_sh = dense_strides[0];
  a.d_st = dense_strides[1];
  a.page_ids = page_ids;
  a.n_ids = n_ids;
  a.num_pages = num_pages;
  a.T = n_tokens;
  a.H = num_heads;
  a.D = head_dim;
  a.bs = block_size;
  return launch_token_copy(scatter, a, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace ukv

using namespace ukv;

extern "C" int ukv_kv_scatter_tokens(void* pool_layer, const int64_t* pool_strides, const void* dense,
                                     const int64_t* dense_strides, const int32_t* page_ids, int n_ids,
                                     int num_pages, int n_tokens, int block_size, int num_heads, int head_dim,
                                     ukv_stream_t stream) {
  return token_copy(true, pool_layer, pool_strides, const_cast<void*>(dense), dense_strides, page_ids, n_ids,
                    num_pages, n_tokens, block_size, num_heads, head_dim, stream);
}

extern "C" int ukv_kv_gather_tokens(const void* pool_layer, const int64_t* pool_strides, void* dense,
                                    const int64_t* dense_strides, const int32_t* page_ids, int n_ids,
                                    int num_pages, int n_tokens, int block_size, int num_heads, int head_dim,
                                    ukv_stream_t stream) {
  return token_copy(false, const_cast<void*>(pool_layer), pool_strides, dense, dense_strides, page_ids, n_ids,
                    num_pages, n_tokens, block_size, num_heads, head_dim, stream);
}

extern "C" int ukv_page_copy(const void* const* src_pools, void* const* dst_pools, int npools,
                             const int64_t* src_strides, const int64_t* dst_strides, const int32_t* src_ids,
                             int64_t src_ids_layer_stride, const int32_t* dst_ids, int64_t dst_ids_layer_stride,
                             int n, int layers, int page_elems, int src_pages, int dst_pages,
                             ukv_stream_t stream) {
  if (n < 0 || layers < 0 || npools < 1 || npools > 2 || page_elems <= 0) return UKV_ERR_INVALID_ARGUMENT;
  if (n == 0 || layers == 0) return UKV_OK;
  if (!src_pools || !dst_pools || !src_strides || !dst_strides || !src_ids || !dst_ids)
    return UKV_ERR_INVALID_ARGUMENT;
  if (page_elems % 8 != 0 || !m8(src_strides[0]) || !m8(src_strides[1]) || !m8(dst_strides[0]) ||
      !m8(dst_strides[1]))
    return UKV_ERR_INVALID_ARGUMENT;
  PageCopyArgs a{};
  for (int p = 0; p < npools; ++p) {
    a.src[p] = static_cast<const uint16_t*>(src_pools[p]);
    a.dst[p] = static_cast<uint16_t*>(dst_pools[p]);
    if (!a.src[p] || !a.dst[p] || !a16(a.src[p]) || !a16(a.dst[p])) return UKV_ERR_INVALID_ARGUMENT;
  }
  a.s_layer = src_strides[0];
  a.s_page = src_strides[1];
  a.d_layer = dst_strides[0];
  a.d_page = dst_strides[1];
  a.src_ids = src_ids;
  a.dst_ids = dst_ids;
  a.src_ids_lstride = src_ids_layer_stride;
  a.dst_ids_lstride = dst_ids_layer_stride;
  a.n = n;
  a.layers = layers;
  a.npools = npools;
  a.page_elems = page_elems;
  a.src_pages = src_pages;
  a.dst_pages = dst_pages;
  if ((int64_t)layers * npools > 65535) return UKV_ERR_INVALID_ARGUMENT;
  const int slices = (page_elems / 8 + kCopyThreads - 1) / kCopyThreads;
  // grid.y is limited to 65535: fold larger n into several launches.
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int j0 = 0; j0 < n; j0 += 65535) {
    PageCopyArgs b = a;
    const int nn = std::min(65535, n - j0);
    b.src_ids = a.src_ids + j0;
    b.dst_ids = a.dst_ids + j0;
    b.n = nn;
    hipLaunchKernelGGL(page_copy_kernel, dim3(slices, nn, layers * npools), dim3(kCopyThreads), 0, s, b);
    if (hipGetLastError() != hipSuccess) return UKV_ERR_LAUNCH;
  }
  return UKV_OK;
}

namespace ukv {

int append_decode_rows(void* k_pool_layer, void* v_pool_layer, const int64_t* k_strides, const int64_t* v_strides,
                       const void* k_new, const void* v_new, const int64_t* new_strides, const int32_t* block_table,
                       int max_blocks, const int32_t* lens, int pos_offset, int32_t* new_lens, int batch,
                       int block_size, int num_heads, int head_dim, int num_pages, ukv_stream_t stream) {
  if (batch < 0 || num_heads <= 0 || head_dim <= 0 || max_blocks < 0 || block_size <= 0)
    return UKV_ERR_INVALID_ARGUMENT;
  if (batch == 0) return UKV_OK;
  if (!k_pool_layer || !v_pool_layer || !k_strides || !v_strides || !k_new || !v_new || !new_strides || !lens ||
      (max_blocks > 0 && !block_table))
    return UKV_ERR_INVALID_ARGUMENT;
  AppendArgs a{};
  a.k_pool = static_cast<uint16_t*>(k_pool_layer);
  a.v_pool = static_cast<uint16_t*>(v_pool_layer);
  a.k_sp = k_strides[0];
  a.k_st = k_strides[1];
  a.k_sh = k_strides[2];
  a.v_sp = v_strides[0];
  a.v_st = v_strides[1];
  a.v_sh = v_strides[2];
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.n_sb = new_strides[0];
  a.n_sh = new_strides[1];
  a.block_table = block_table;
  a.max_blocks = max_blocks;
  a.old_lens = lens;
  a.pos_offset = pos_offset;
  a.new_lens = new_lens;
  a.B = batch;
  a.H = num_heads;
  a.D = head_dim;
  a.num_pages = num_pages;
  a.bs = block_size;
  a.vec = head_dim % 8 == 0 && a16(k_pool_layer) && a16(v_pool_layer) && a16(k_new) && a16(v_new) &&
          m8(a.k_sp) && m8(a.k_st) && m8(a.k_sh) && m8(a.v_sp) && m8(a.v_st) && m8(a.v_sh) && m8(a.n_sb) &&
          m8(a.n_sh);
  hipLaunchKernelGGL(kv_append_kernel, dim3(batch), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}

}  // namespace ukv

extern "C" int ukv_kv_append(void* k_pool_layer, void* v_pool_layer, const int64_t* k_strides,
                             const int64_t* v_strides, const void* k_new, const void* v_new,
                             const int64_t* new_strides, const int32_t* block_table, int max_blocks,
                             const int32_t* old_lens, int32_t* new_lens, int batch, int block_size,
                             int num_heads, int head_dim, int num_pages, ukv_stream_t stream) {
  return append_decode_rows(k_pool_layer, v_pool_layer, k_strides, v_strides, k_new, v_new, new_strides,
                            block_table, max_blocks, old_lens, 0, new_lens, batch, block_size, num_heads, head_dim,
                            num_pages, stream);
}

extern "C" int ukv_decode_prologue(int32_t* block_table, int max_blocks, int batch, const int32_t* lens_in,
                                   int32_t* lens_out, const int32_t* new_pages, int n_new, ukv_stream_t stream) {
  if (batch < 0 || max_blocks < 0 || n_new < 0) return UKV_ERR_INVALID_ARGUMENT;
  if (n_new > 0 && (!new_pages || !block_table)) return UKV_ERR_INVALID_ARGUMENT;
  if (lens_out && batch > 0 && !lens_in) return UKV_ERR_INVALID_ARGUMENT;
  // The triples are host memory: validate every one before launching anything.
  for (int i = 0; i < n_new; ++i) {
    const int32_t row = new_pages[3 * i], col = new_pages[3 * i + 1];
    if (row < 0 || row >= batch || col < 0 || col >= max_blocks) return UKV_ERR_INVALID_ARGUMENT;
  }
  const bool lens = lens_out && batch > 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int i0 = 0; i0 < n_new || (i0 == 0 && lens); i0 += kPrologueMax) {
    PrologueArgs a{};
    a.bt = block_table;
    a.max_blocks = max_blocks;
    a.B = batch;
    a.lens_in = lens_in;
    a.lens_out = (i0 == 0 && lens) ? lens_out : nullptr;
    a.n = std::min(kPrologueMax, std::max(0, n_new - i0));
    std::copy(new_pages + 3 * i0, new_pages + 3 * (i0 + a.n), a.trip);
    hipLaunchKernelGGL(decode_prologue_kernel, dim3(1), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return UKV_ERR_LAUNCH;
  }
  return UKV_OK;
}
