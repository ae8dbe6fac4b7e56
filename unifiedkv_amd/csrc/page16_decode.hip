// Page16 paged decode attention for gfx950 (MI355X).
//
// Semantics follow core/page16_native.py:17-80 (BP-KV): for every sequence b and
// q head h, attend over tokens t < seqlens[b] whose K/V rows live at
// cache[block_table[b, t/16], t%16, h/n_rep, :], fp32 online softmax, output
// acc/l rounded to the input dtype.
//
// Work decomposition (split-K / flash-decoding):
//   * grid (chunk, sequence, kv-group block). One workgroup streams
//     `chunk_pages` consecutive pages of one sequence for up to eight KV heads,
//     one wave per KV head, so a workgroup reads each 32 KiB K page and 32 KiB V
//     page of its chunk whole, and every KV byte is read exactly once for all
//     n_rep q heads that share it (GQA packing).
//   * QK^T on the matrix core: one v_mfma_f32_16x16x32 per 32 head dims with
//     A = the wave's q heads (rows, zero-padded to 16) and B = the page's 16
//     K rows (columns). K rows are loaded straight from HBM into the B-operand
//     layout, 16 bytes per lane per step.
//   * online softmax in log2 units (exp2 with the log2(e) factor folded into
//     the scale) with 16-lane DPP row reductions.
//   * P.V in fp32 on the VALU: V rows are loaded 16 bytes per lane with each
//     row read by D/8 consecutive lanes; p and the rescale factor reach those
//     lanes through a small per-wave LDS buffer.
//   * a second kernel merges the per-chunk (m, l, acc) partials (log-sum-exp).
//
// A reference-faithful scalar kernel (natural exp, one workgroup per (b, h))
// serves shapes the split kernel is not instantiated for (head_dim not in
// {64, 128, 256}, n_rep > 16, or rows not 16-byte aligned).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "ukv_common.h"

namespace ukv {

struct DecodeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* bt;
  const int32_t* lens;
  uint16_t* out;
  float* part_o;    // [B][max_chunks][Hq][D]
  float2* part_ml;  // [B][max_chunks][Hq]: (running max in log2 units, sum of exp2)
  int64_t q_sb, q_sh;
  int64_t k_sp, k_st, k_sh;
  int64_t v_sp, v_st, v_sh;
  int B, Hq, n_rep, n_groups, D, max_blocks, num_pages;
  int chunk_pages, max_chunks;
  float scale;       // natural-log units (scalar kernel)
  float scale_log2;  // scale * log2(e) (split kernel)
};

__device__ __forceinline__ int clamp_len(int L, int max_blocks) {
  const int cap = max_blocks * 16;
  return L < 0 ? 0 : (L > cap ? cap : L);
}

// Orders LDS traffic of one wave: writes before the barrier are visible to
// every lane of the wave after it (LDS executes a wave's requests in order).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int DT, int D, int NREP>
__global__ void __launch_bounds__(512) page16_split_kernel(const DecodeArgs a) {
  constexpr int STEPS = D / 32;  // MFMA k-steps over the head dimension
  constexpr int RL = D / 8;      // lanes per V row (8 dims per lane)
  constexpr int TG = 64 / RL;    // V token groups per wave
  constexpr int TPL = 16 / TG;   // V tokens per lane per page
  constexpr int NP = NREP < 4 ? 4 : NREP;
  constexpr int HG4 = (NREP + 3) / 4;       // QK row groups holding real q heads
  constexpr int BUF = 16 * NP + NP;         // p[16][NP] followed by alpha[NP]
  static_assert(TG * TPL == 16, "V layout must cover a page");

  __shared__ __attribute__((aligned(16))) float lds_all[8 * 2 * BUF];

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int g = blockIdx.z * (blockDim.x >> 6) + wv;
  if (g >= a.n_groups) return;  // whole wave leaves; no workgroup barrier below
  const int b = blockIdx.y;
  const int chunk = blockIdx.x;

  const int L = clamp_len(a.lens[b], a.max_blocks);
  const int n_pages = (L + 15) >> 4;
  const int p0 = chunk * a.chunk_pages;
  if (p0 >= n_pages) return;
  const int p1 = min(p0 + a.chunk_pages, n_pages);

  float* lds = lds_all + wv * 2 * BUF;
  const int j = lane & 15;   // QK layout: token column / q row
  const int kg = lane >> 4;  // QK layout: k-slot group
  const int rl = lane % RL;  // V layout: dims 8*rl .. 8*rl+7
  const int tg = lane / RL;  // V layout: tokens tg*TPL .. tg*TPL+TPL-1

  const int qh0 = g * a.n_rep;
  const int n_here = min(a.n_rep, a.Hq - qh0);

  // A operand: row j = q head qh0 + j; k-slot group kg at step s covers dims
  // 32*s + 8*kg .. +7 (the same dims the K rows supply below).
  u32x4 qa[STEPS];
  {
    const bool live = j < n_here;
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(qh0 + (live ? j : 0)) * a.q_sh + 8 * kg;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) qa[s] = live ? ld16(qp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
  }

  const int32_t* btrow = a.bt + (int64_t)b * a.max_blocks;
  const uint16_t* kbase = a.k + (int64_t)j * a.k_st + (int64_t)g * a.k_sh + 8 * kg;
  const uint16_t* vbase = a.v + (int64_t)(tg * TPL) * a.v_st + (int64_t)g * a.v_sh + 8 * rl;

  float m[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = kNegFltMax;
    l[r] = 0.f;
  }
  float acc[NREP][8];
#pragma unroll
  for (int h = 0; h < NREP; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;

  auto load_page = [&](int p, u32x4 (&kr)[STEPS], u32x4 (&vr)[TPL], int& nv) {
    int bid = btrow[p];
    const bool ok = (unsigned)bid < (unsigned)a.num_pages;
    bid = ok ? bid : 0;
    nv = ok ? min(16, L - 16 * p) : 0;
    const uint16_t* kp = kbase + (int64_t)bid * a.k_sp;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) kr[s] = ld16(kp + 32 * s);
    const uint16_t* vp = vbase + (int64_t)bid * a.v_sp;
#pragma unroll
    for (int i = 0; i < TPL; ++i) vr[i] = ld16(vp + (int64_t)i * a.v_st);
  };

  auto process_page = [&](const u32x4 (&kr)[STEPS], u32x4 (&vr)[TPL], int nv, float* buf) {
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) sacc = mfma16x16x32<DT>(qa[s], kr[s], sacc);

    // lane (j, kg) holds the score of q head 4*kg + r against token j.
    float pr[4], al[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s2 = (j < nv) ? sacc[r] * a.scale_log2 : -INFINITY;
      const float mn = fmaxf(m[r], row_max16(s2));
      al[r] = fast_exp2(m[r] - mn);
      pr[r] = fast_exp2(s2 - mn);
      l[r] = l[r] * al[r] + row_sum16(pr[r]);
      m[r] = mn;
    }
    if (kg < HG4) {
      *reinterpret_cast<f32x4*>(buf + j * NP + 4 * kg) = f32x4{pr[0], pr[1], pr[2], pr[3]};
      if (j == 0) *reinterpret_cast<f32x4*>(buf + 16 * NP + 4 * kg) = f32x4{al[0], al[1], al[2], al[3]};
    }
    wave_lds_sync();

    float alpha[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) alpha[h] = buf[16 * NP + h];
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= alpha[h];

#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      const int t = tg * TPL + i;
      u32x4 w = vr[i];
      if (t >= nv) w = u32x4{0u, 0u, 0u, 0u};  // masked rows may hold non-finite junk
      float vf[8];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        vf[2 * c] = Elem<DT>::lo(w[c]);
        vf[2 * c + 1] = Elem<DT>::hi(w[c]);
      }
      const float* prow = buf + t * NP;
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        const float ph = prow[h];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(ph, vf[e], acc[h][e]);
      }
    }
    wave_lds_sync();
  };

  // Software pipeline: the loads of page p+1 are in flight while page p is
  // reduced. Two register sets and two LDS buffers alternate.
  u32x4 kA[STEPS], vA[TPL], kB[STEPS], vB[TPL];
  int nvA, nvB;
  load_page(p0, kA, vA, nvA);
  int p = p0;
  for (; p + 1 < p1; p += 2) {
    load_page(p + 1, kB, vB, nvB);
    process_page(kA, vA, nvA, lds);
    if (p + 2 < p1) load_page(p + 2, kA, vA, nvA);
    process_page(kB, vB, nvB, lds + BUF);
  }
  if (p < p1) process_page(kA, vA, nvA, lds);

  // Sum the V-layout token groups.
#pragma unroll
  for (int o = RL; o < 64; o <<= 1)
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] += __shfl_xor(acc[h][e], o);

  const int64_t slot = ((int64_t)b * a.max_chunks + chunk) * a.Hq + qh0;
  if (tg == 0) {
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      if (h < n_here) {
        f32x4* dst = reinterpret_cast<f32x4*>(a.part_o + (slot + h) * D + 8 * rl);
        dst[0] = f32x4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
        dst[1] = f32x4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
      }
    }
  }
  if (j == 0 && kg < HG4) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * kg + r;
      if (h < n_here) a.part_ml[slot + h] = make_float2(m[r], l[r]);
    }
  }
}

// Merges the chunk partials of one (sequence, q head): log-sum-exp in log2 units.
template <int DT>
__global__ void __launch_bounds__(64) page16_combine_kernel(const DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int L = clamp_len(a.lens[b], a.max_blocks);
  const int n_pages = (L + 15) >> 4;
  const int n_chunks = (n_pages + a.chunk_pages - 1) / a.chunk_pages;
  const int64_t base = (int64_t)b * a.max_chunks * a.Hq + h;

  float M = -INFINITY;
  for (int c = 0; c < n_chunks; ++c) M = fmaxf(M, a.part_ml[base + (int64_t)c * a.Hq].x);
  float den = 0.f;
  for (int c = 0; c < n_chunks; ++c) {
    const float2 ml = a.part_ml[base + (int64_t)c * a.Hq];
    den += ml.y * exp2f(ml.x - M);
  }
  uint16_t* orow = a.out + ((int64_t)b * a.Hq + h) * a.D;
  for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
    float num = 0.f;
    for (int c = 0; c < n_chunks; ++c) {
      const int64_t s = base + (int64_t)c * a.Hq;
      num += exp2f(a.part_ml[s].x - M) * a.part_o[s * a.D + d];
    }
    orow[d] = Elem<DT>::from_float(n_chunks > 0 ? num / den : NAN);
  }
}

// One workgroup per (q head, sequence); the same arithmetic as the reference
// Triton program: natural exp, -FLT_MAX for masked scores, page loop in order.
template <int DT>
__global__ void __launch_bounds__(256) page16_scalar_kernel(const DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int g = h / a.n_rep;
  const int tid = threadIdx.x;
  const int t = tid >> 4;
  const int sub = tid & 15;
  __shared__ float qs[256];
  __shared__ float ss[16];

  const uint16_t* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  for (int d = tid; d < a.D; d += blockDim.x) qs[d] = Elem<DT>::one(qrow[d]);
  __syncthreads();

  const int L = clamp_len(a.lens[b], a.max_blocks);
  const int n_pages = (L + 15) >> 4;
  const int d = tid;
  float m = kNegFltMax, l = 0.f, acc = 0.f;
  for (int p = 0; p < n_pages; ++p) {
    int bid = a.bt[(int64_t)b * a.max_blocks + p];
    const bool ok = (unsigned)bid < (unsigned)a.num_pages;
    bid = ok ? bid : 0;
    const int nv = ok ? min(16, L - 16 * p) : 0;
    float part = 0.f;
    if (t < nv) {
      const uint16_t* krow = a.k + (int64_t)bid * a.k_sp + (int64_t)t * a.k_st + (int64_t)g * a.k_sh;
      for (int dd = sub; dd < a.D; dd += 16) part += Elem<DT>::one(krow[dd]) * qs[dd];
    }
    part = row_sum16(part);
    if (sub == 0) ss[t] = (t < nv) ? part * a.scale : kNegFltMax;
    __syncthreads();
    float mx = kNegFltMax;
    for (int tt = 0; tt < 16; ++tt) mx = fmaxf(mx, ss[tt]);
    const float mn = fmaxf(m, mx);
    const float alpha = expf(m - mn);
    float psum = 0.f, pv = 0.f;
    for (int tt = 0; tt < 16; ++tt) {
      const float pt = (tt < nv) ? expf(ss[tt] - mn) : 0.f;
      psum += pt;
      if (d < a.D && tt < nv)
        pv += pt * Elem<DT>::one(a.v[(int64_t)bid * a.v_sp + (int64_t)tt * a.v_st + (int64_t)g * a.v_sh + d]);
    }
    l = l * alpha + psum;
    acc = acc * alpha + pv;
    m = mn;
    __syncthreads();
  }
  if (d < a.D) a.out[((int64_t)b * a.Hq + h) * a.D + d] = Elem<DT>::from_float(acc / l);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

constexpr int kMinChunkPages = 4;
constexpr int kMaxChunkPages = 64;

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev < 64) cached[dev] = cus;
  return cus;
}

// Pages per split-K chunk: about four workgroups per CU over the whole batch,
// overridable with UKV_PAGE16_CHUNK_PAGES for launch-shape sweeps.
int chunk_pages_for(int batch, int max_blocks) {
  const char* env = std::getenv("UKV_PAGE16_CHUNK_PAGES");
  if (env && *env) {
    const int v = std::atoi(env);
    if (v > 0) return v;
  }
  const long long total = (long long)batch * (long long)std::max(max_blocks, 1);
  const long long target = 4LL * device_cu_count();
  long long c = (total + target - 1) / target;
  c = std::max<long long>(kMinChunkPages, std::min<long long>(kMaxChunkPages, c));
  return (int)c;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct WorkspaceLayout {
  size_t part_o_off, part_ml_off, total;
  int chunk_pages, max_chunks;
};

WorkspaceLayout workspace_layout(int batch, int hq, int d, int max_blocks) {
  WorkspaceLayout w{};
  w.chunk_pages = chunk_pages_for(batch, max_blocks);
  w.max_chunks = std::max(1, (std::max(max_blocks, 0) + w.chunk_pages - 1) / w.chunk_pages);
  const size_t slots = (size_t)batch * w.max_chunks * hq;
  w.part_o_off = 0;
  w.part_ml_off = align256(slots * d * sizeof(float));
  w.total = w.part_ml_off + align256(slots * sizeof(float2));
  return w;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT, int D, int NREP>
void launch_split(const DecodeArgs& a, hipStream_t stream) {
  const int waves = std::min(8, a.n_groups);
  const dim3 grid(a.max_chunks, a.B, (a.n_groups + waves - 1) / waves);
  hipLaunchKernelGGL((page16_split_kernel<DT, D, NREP>), grid, dim3(64 * waves), 0, stream, a);
}

template <int DT, int D>
bool dispatch_nrep(const DecodeArgs& a, hipStream_t stream) {
  if (a.n_rep <= 1) launch_split<DT, D, 1>(a, stream);
  else if (a.n_rep <= 2) launch_split<DT, D, 2>(a, stream);
  else if (a.n_rep <= 4) launch_split<DT, D, 4>(a, stream);
  else if (a.n_rep <= 8) launch_split<DT, D, 8>(a, stream);
  else if (a.n_rep <= 16) launch_split<DT, D, 16>(a, stream);
  else return false;
  return true;
}

template <int DT>
bool dispatch_split(const DecodeArgs& a, hipStream_t stream) {
  switch (a.D) {
    case 64: return dispatch_nrep<DT, 64>(a, stream);
    case 128: return dispatch_nrep<DT, 128>(a, stream);
    case 256: return dispatch_nrep<DT, 256>(a, stream);
    default: return false;
  }
}

}  // namespace
}  // namespace ukv

using namespace ukv;

extern "C" size_t ukv_page16_workspace_bytes(int batch, int num_q_heads, int head_dim, int max_blocks) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  return workspace_layout(batch, num_q_heads, head_dim, max_blocks).total;
}

extern "C" int ukv_page16_decode(const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* block_table, const int32_t* seqlens, void* out, int batch,
                                 int num_q_heads, int num_kv_heads, int head_dim, int n_rep, int max_blocks,
                                 int num_pages, const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, float softmax_scale, int dtype, void* workspace,
                                 size_t workspace_bytes, ukv_stream_t stream_handle) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0) return UKV_ERR_EMPTY;
  if (head_dim > 256) return UKV_ERR_HEAD_DIM;
  if (dtype != UKV_DTYPE_F16 && dtype != UKV_DTYPE_BF16) return UKV_ERR_DTYPE;
  if (num_kv_heads <= 0 || n_rep < 1) return UKV_ERR_GQA;
  const int n_groups = (num_q_heads + n_rep - 1) / n_rep;
  if (n_groups > num_kv_heads) return UKV_ERR_GQA;
  if (max_blocks < 0 || num_pages < 0) return UKV_ERR_INVALID_ARGUMENT;
  if (!q || !out || !seqlens || !q_strides || !k_strides || !v_strides) return UKV_ERR_INVALID_ARGUMENT;
  if (max_blocks > 0 && (!block_table || !k_cache || !v_cache || num_pages <= 0)) return UKV_ERR_INVALID_ARGUMENT;

  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
  DecodeArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k_cache);
  a.v = static_cast<const uint16_t*>(v_cache);
  a.bt = block_table;
  a.lens = seqlens;
  a.out = static_cast<uint16_t*>(out);
  a.q_sb = q_strides[0];
  a.q_sh = q_strides[1];
  a.k_sp = k_strides[0];
  a.k_st = k_strides[1];
  a.k_sh = k_strides[2];
  a.v_sp = v_strides[0];
  a.v_st = v_strides[1];
  a.v_sh = v_strides[2];
  a.B = batch;
  a.Hq = num_q_heads;
  a.n_rep = n_rep;
  a.n_groups = n_groups;
  a.D = head_dim;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * kLog2e;

  const bool strides_ok = (a.q_sb % 8 == 0) && (a.q_sh % 8 == 0) && (a.k_sp % 8 == 0) && (a.k_st % 8 == 0) &&
                          (a.k_sh % 8 == 0) && (a.v_sp % 8 == 0) && (a.v_st % 8 == 0) && (a.v_sh % 8 == 0);
  const bool fast = (head_dim == 64 || head_dim == 128 || head_dim == 256) && n_rep <= 16 && strides_ok &&
                    aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out) && max_blocks > 0;

  if (fast) {
    const WorkspaceLayout w = workspace_layout(batch, num_q_heads, head_dim, max_blocks);
    if (!workspace || workspace_bytes < w.total || !aligned16(workspace)) return UKV_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    a.part_o = reinterpret_cast<float*>(ws + w.part_o_off);
    a.part_ml = reinterpret_cast<float2*>(ws + w.part_ml_off);
    a.chunk_pages = w.chunk_pages;
    a.max_chunks = w.max_chunks;
    const bool launched =
        dtype == UKV_DTYPE_BF16 ? dispatch_split<UKV_DTYPE_BF16>(a, stream) : dispatch_split<UKV_DTYPE_F16>(a, stream);
    if (!launched) return UKV_ERR_LAUNCH;
    if (hipGetLastError() != hipSuccess) return UKV_ERR_LAUNCH;
    const dim3 grid(num_q_heads, batch);
    if (dtype == UKV_DTYPE_BF16)
      hipLaunchKernelGGL(page16_combine_kernel<UKV_DTYPE_BF16>, grid, dim3(64), 0, stream, a);
    else
      hipLaunchKernelGGL(page16_combine_kernel<UKV_DTYPE_F16>, grid, dim3(64), 0, stream, a);
  } else {
    const dim3 grid(num_q_heads, batch);
    if (dtype == UKV_DTYPE_BF16)
      hipLaunchKernelGGL(page16_scalar_kernel<UKV_DTYPE_BF16>, grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(page16_scalar_kernel<UKV_DTYPE_F16>, grid, dim3(256), 0, stream, a);
  }
  if (hipGetLastError() != hipSuccess) return UKV_ERR_LAUNCH;
  return UKV_OK;
}
