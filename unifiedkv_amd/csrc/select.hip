// Retain-set selection for block compression (gfx950): per row, the k best pages by score.
//
// The reference ranks mid-segment blocks with torch.topk and sorts the winners
// (core/scheduler.py:613-616, core/compress.py:141-142); torch leaves the order
// of equal scores unspecified, so this build fixes it: higher score first, then
// lower index; NaN ranks above every number (as torch.topk treats it). The
// winners are written in ascending index order.
//
// One 256-thread workgroup per row. Each element gets a unique 64-bit key,
//   key = (~orderable(score) << 32) | index,
// so "k smallest keys" is exactly the selection. A radix select over the 64
// key bits (8 passes of 8-bit digits, LDS histograms) finds the k-th smallest
// key T; the winners are the elements with key <= T, compacted in index order
// with a block-wide prefix sum. Any row length works; the row is re-read from
// global memory (L2) on each pass.
#include "ukv_common.h"

namespace ukv {

__device__ __forceinline__ uint64_t select_key(float s, int idx) {
  uint32_t u = __float_as_uint(s);
  if (s != s) u = 0x7fc00000u;  // canonical NaN ranks highest
  if (u == 0x80000000u) u = 0u;  // -0 equals +0: the tie goes to the lower index
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // ascending with the float value
  return (uint64_t(~ord) << 32) | uint32_t(idx);
}

// Exclusive prefix sum of one value per thread over a 256-thread block.
__device__ __forceinline__ int block_exclusive_scan_256(int v, int* sh) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[wv] = x;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wv; ++w) base += sh[w];
  __syncthreads();
  return base + x - v;
}

__global__ void __launch_bounds__(256) select_topk_kernel(const float* __restrict__ scores, int64_t row_stride,
                                                          const int32_t* __restrict__ row_n,
                                                          const int32_t* __restrict__ row_k, int n_max, int k_max,
                                                          int32_t* __restrict__ out, int64_t out_stride) {
  __shared__ unsigned hist[256];
  __shared__ int scan_sh[4];
  __shared__ uint64_t s_prefix;
  __shared__ int s_need;

  const int row = blockIdx.x;
  const float* sc = scores + (int64_t)row * row_stride;
  int32_t* o = out + (int64_t)row * out_stride;
  int n = row_n ? row_n[row] : n_max;
  n = n < 0 ? 0 : (n > n_max ? n_max : n);
  int k = row_k ? row_k[row] : k_max;
  k = k < 0 ? 0 : (k > n ? n : k);
  k = k > k_max ? k_max : k;

  for (int i = k + threadIdx.x; i < k_max; i += blockDim.x) o[i] = -1;
  if (k == 0) return;

  // Radix select of the k-th smallest key: prefix holds the decided high bits.
  if (threadIdx.x == 0) {
    s_prefix = 0;
    s_need = k;  // rank (1-based) of the wanted key among keys matching the prefix
  }
  uint64_t T = ~uint64_t(0);
  if (k < n) {
    for (int pass = 0; pass < 8; ++pass) {
      const int shift = 56 - 8 * pass;
      const uint64_t hi_mask = pass == 0 ? 0 : (~uint64_t(0) << (shift + 8));
      hist[threadIdx.x] = 0;
      __syncthreads();
      const uint64_t prefix = s_prefix;
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t key = select_key(sc[i], i);
        if ((key & hi_mask) == prefix) atomicAdd(&hist[(key >> shift) & 0xff], 1u);
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        int need = s_need;
        int d = 0;
        for (; d < 256; ++d) {
          if ((int)hist[d] >= need) break;
          need -= (int)hist[d];
        }
        s_prefix = prefix | (uint64_t(d) << shift);
        s_need = need;
      }
      __syncthreads();
    }
    T = s_prefix;  // keys are unique, so the full 64-bit prefix is the k-th key
  }

  // Winners (key <= T) in ascending index order.
  int written = 0;
  for (int base = 0; base < n; base += blockDim.x) {
    const int i = base + threadIdx.x;
    const int flag = (i < n) && (select_key(sc[i], i) <= T);
    const int pos = written + block_exclusive_scan_256(flag, scan_sh);
    if (flag) o[pos] = i;
    const int total = __syncthreads_count(flag);
    written += total;
  }
}

}  // namespace ukv

using namespace ukv;

// scores float32 [rows][row_stride >= n_max]; row_n / row_k optional int32 [rows] device arrays
// (NULL: n_max / k_max for every row); out int32 [rows][out_stride >= k_max].
extern "C" int ukv_select_topk(const float* scores, int64_t row_stride, const int32_t* row_n, const int32_t* row_k,
                               int rows, int n_max, int k_max, int32_t* out, int64_t out_stride,
                               ukv_stream_t stream) {
  if (rows < 0 || n_max < 0 || k_max < 0 || row_stride < n_max || out_stride < k_max) return UKV_ERR_INVALID_ARGUMENT;
  if (rows == 0 || k_max == 0) return UKV_OK;
  if (!scores || !out) return UKV_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(select_topk_kernel, dim3(rows), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), scores,
                     row_stride, row_n, row_k, n_max, k_max, out, out_stride);
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}
