// Chunked prefill attention over the paged pool (gfx950, bf16/fp16 MFMA).
//
// Semantics: for sequence b with kv_lens[b] keys resident in pages (the
// prefix plus this chunk) and C_b = cu_q[b+1] - cu_q[b] chunk queries, query i
// sits at absolute position P_b + i, P_b = kv_lens[b] - C_b, and attends to
// keys 0 .. P_b + i (causal, aligned to the bottom right) - what the
// reference's chunked prefill computes through HF attention over the past KV
// (core/engine.py:1826-1854, core/chunked_prefill.py:9-33) and what
// flash_attn_varlen_func(causal=True) computes for a single chunk
// (core/varlen.py:19-42). The reference has no paged prefill; here the keys
// are read from 16-token pages through the block table, and
// ukv_kv_write_varlen first writes the chunk's own K/V into its pages.
//
// Kernel: grid (query blocks, KV groups, sequences), 4 waves. A workgroup takes
// QW = 4 * CB * (16 / n_rep) consecutive queries of one KV group. Within a
// wave, an MFMA column is a (query, q head) pair: 16 / n_rep queries times the
// n_rep q heads of the group, so one K/V read serves the whole GQA group.
//   * key tiles of 32 keys (two pages) are staged in LDS (double buffered, rows
//     padded to 272 B so 16 lanes reading 16 rows hit distinct banks) and
//     shared by the 4 waves;
//   * S^T = K Q^T on v_mfma_f32_16x16x32 (A = 16 keys x 32 dims from LDS,
//     B = the wave's q columns held in registers); lane l ends with keys
//     4*(l/16) + r of column l % 16;
//   * online softmax per column in log2 units, causal and validity masks, and
//     the running max moved only when a score exceeds it by 2^8 (wave vote);
//   * P.V on v_mfma_f32_16x16x32 (bf16 P as a rounded value plus its
//     residual, two MFMAs; fp16 P rounded once): the S^T layout is
//     already P's A-operand layout (k-slots = the lane's 8 keys of the tile);
//     V's B operands come from 8 LDS row reads per lane regrouped with
//     v_perm_b32.
#include <algorithm>
#include <cmath>

#include "ukv_common.h"

namespace ukv {

struct PrefillArgs {
  const uint16_t* q;  // [total_q][Hq][D]
  uint16_t* out;      // [total_q][Hq][D] contiguous
  const uint16_t* k;  // one pool layer [N][16][Hkv][D]
  const uint16_t* v;
  int64_t q_st, q_sh;
  int64_t k_sp, k_st, k_sh;
  int64_t v_sp, v_st, v_sh;
  const int32_t* bt;
  const int32_t* cu_q;     // [B+1]
  const int32_t* kv_lens;  // [B] keys per sequence, the chunk included
  int B, Hq, n_rep, n_groups, D, max_blocks, num_pages;
  float scale, scale_log2;
};

__device__ __forceinline__ int kv_len_of(const PrefillArgs& a, int b) {
  const int cap = a.max_blocks * 16;
  const int L = a.kv_lens[b];
  return L < 0 ? 0 : (L > cap ? cap : L);
}

template <int DT> __device__ __forceinline__ uint32_t pack2(float x0, float x1);
template <> __device__ __forceinline__ uint32_t pack2<UKV_DTYPE_BF16>(float x0, float x1) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, bf16x2));
}
template <> __device__ __forceinline__ uint32_t pack2<UKV_DTYPE_F16>(float x0, float x1) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, f16x2));
}

#ifndef UKV_PREFILL_SPLIT_P
#define UKV_PREFILL_SPLIT_P 1
#endif

constexpr int kTileKeys = 32;
constexpr int kRowPad = 136;  // LDS row pitch in 16-bit elements (128 + 8)

template <int DT, int CB>
__global__ void __launch_bounds__(256) paged_prefill_kernel(const PrefillArgs a) {
  constexpr int D = 128;
  constexpr int STEPS = D / 32;
  constexpr float kTau = 8.f;
  constexpr bool kSplitP = DT == UKV_DTYPE_BF16 && UKV_PREFILL_SPLIT_P;
  __shared__ __attribute__((aligned(16))) uint16_t k_s[2][kTileKeys][kRowPad];
  __shared__ __attribute__((aligned(16))) uint16_t v_s[2][kTileKeys][kRowPad];
  __shared__ int valid_s[2][kTileKeys];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int i16 = lane & 15;
  const int kg = lane >> 4;
  const int g = blockIdx.y;
  const int b = blockIdx.z;

  const int qpb = 16 / a.n_rep;  // queries per column block
  const int qw = 4 * CB * qpb;   // queries per workgroup
  const int q_begin = a.cu_q[b];
  const int C = a.cu_q[b + 1] - q_begin;
  const int q0 = blockIdx.x * qw;
  if (q0 >= C) return;  // whole workgroup
  const int Lk = kv_len_of(a, b);
  const int P0 = Lk - C;  // keys before the chunk
  const int q_last = min(C, q0 + qw) - 1;
  const int kend = max(0, min(Lk, P0 + q_last + 1));
  const int n_tiles = (kend + kTileKeys - 1) / kTileKeys;

  // This lane's columns: (query, head) of column i16 in each column block.
  const int head_local = i16 % a.n_rep;
  const int head = g * a.n_rep + head_local;
  int qpos[CB];  // absolute position of the column's query, or -1 if the column is unused
  u32x4 qb[CB][STEPS];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int qi = q0 + (wv * CB + cb) * qpb + i16 / a.n_rep;
    const bool live = qi < C && head < a.Hq;
    qpos[cb] = live ? P0 + qi : -1;
    const uint16_t* qp = a.q + (int64_t)(q_begin + (live ? qi : 0)) * a.q_st + (int64_t)(live ? head : 0) * a.q_sh +
                         8 * kg;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) qb[cb][s] = live ? ld16(qp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
  }

  float m_ref[CB], lsum[CB];
  f32x4 o[CB][8];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    m_ref[cb] = kNegFltMax;
    lsum[cb] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[cb][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Tile loader: thread t moves 16-byte chunk t % 16 of rows t / 16 and
  // 16 + t / 16 of the K and the V tile (rows = keys).
  const int lrow = tid >> 4;
  const int lchunk = tid & 15;
  const int32_t* btrow = a.bt + (int64_t)b * a.max_blocks;
  u32x4 ldk[2], ldv[2];
  int ldok[2];
  auto fetch_tile = [&](int t) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int key = t * kTileKeys + h * 16 + lrow;
      int page = key < Lk ? btrow[key >> 4] : -1;
      const bool ok = (unsigned)page < (unsigned)a.num_pages;
      ldok[h] = ok;
      page = ok ? page : 0;
      const int64_t kt = (int64_t)page * a.k_sp + (int64_t)(key & 15) * a.k_st + (int64_t)g * a.k_sh + 8 * lchunk;
      const int64_t vt = (int64_t)page * a.v_sp + (int64_t)(key & 15) * a.v_st + (int64_t)g * a.v_sh + 8 * lchunk;
      ldk[h] = ok ? ld16(a.k + kt) : u32x4{0u, 0u, 0u, 0u};
      ldv[h] = ok ? ld16(a.v + vt) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      *reinterpret_cast<u32x4*>(&k_s[buf][h * 16 + lrow][8 * lchunk]) = ldk[h];
      *reinterpret_cast<u32x4*>(&v_s[buf][h * 16 + lrow][8 * lchunk]) = ldv[h];
      if (lchunk == 0) valid_s[buf][h * 16 + lrow] = ldok[h];
    }
  };

  if (n_tiles > 0) {
    fetch_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) fetch_tile(t + 1);  // in flight during this tile's math
    const int key0 = t * kTileKeys;

    // S^T[key][column] for the tile's two 16-key blocks and every column block.
    f32x4 sacc[2][CB];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) sacc[kb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(&k_s[buf][kb * 16 + i16][32 * s + 8 * kg]);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) sacc[kb][cb] = mfma16x16x32<DT>(ka, qb[cb][s], sacc[kb][cb]);
      }
    }
    int kvalid[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) kvalid[kb][r] = valid_s[buf][kb * 16 + 4 * kg + r];

    // V B-operands: lane (i16, kg) reads keys 4kg..4kg+3 and 16+4kg.. of dims 8*i16..+7.
    u32x4 vr[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) vr[kb][r] = *reinterpret_cast<const u32x4*>(&v_s[buf][kb * 16 + 4 * kg + r][8 * i16]);

#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      float s2[2][4];
      float mloc = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = key0 + kb * 16 + 4 * kg + r;
          const bool ok = kvalid[kb][r] && key <= qpos[cb];
          s2[kb][r] = ok ? sacc[kb][cb][r] * a.scale_log2 : -INFINITY;
          mloc = fmaxf(mloc, s2[kb][r]);
        }
      if (__any(mloc > m_ref[cb] + kTau)) {
        float mcol = fmaxf(mloc, __shfl_xor(mloc, 16));
        mcol = fmaxf(mcol, __shfl_xor(mcol, 32));
        const float m_new = fmaxf(m_ref[cb], mcol);
        const float alpha = fast_exp2(m_ref[cb] - m_new);
        lsum[cb] *= alpha;
        m_ref[cb] = m_new;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * kg + r);
#pragma unroll
          for (int e = 0; e < 8; ++e) o[cb][e][r] *= ar;
        }
      }
      float p[2][4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[kb][r] = fast_exp2(s2[kb][r] - m_ref[cb]);
          lsum[cb] += p[kb][r];
        }
      const u32x4 pa = {pack2<DT>(p[0][0], p[0][1]), pack2<DT>(p[0][2], p[0][3]), pack2<DT>(p[1][0], p[1][1]),
                        pack2<DT>(p[1][2], p[1][3])};
      // bf16 keeps 8 significant bits of P: a second MFMA adds the rounding
      // residual so that few-key rows stay within the fp32-accumulation
      // tolerance (fp16 P keeps 11 bits and needs no residual).
      u32x4 pl = {0u, 0u, 0u, 0u};
      if constexpr (kSplitP) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float r0 = p[c >> 1][2 * (c & 1)] - __uint_as_float(pa[c] << 16);
          const float r1 = p[c >> 1][2 * (c & 1) + 1] - __uint_as_float(pa[c] & 0xffff0000u);
          pl[c] = pack2<DT>(r0, r1);
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 blo = {__builtin_amdgcn_perm(vr[0][1][c], vr[0][0][c], 0x05040100u),
                           __builtin_amdgcn_perm(vr[0][3][c], vr[0][2][c], 0x05040100u),
                           __builtin_amdgcn_perm(vr[1][1][c], vr[1][0][c], 0x05040100u),
                           __builtin_amdgcn_perm(vr[1][3][c], vr[1][2][c], 0x05040100u)};
        const u32x4 bhi = {__builtin_amdgcn_perm(vr[0][1][c], vr[0][0][c], 0x07060302u),
                           __builtin_amdgcn_perm(vr[0][3][c], vr[0][2][c], 0x07060302u),
                           __builtin_amdgcn_perm(vr[1][1][c], vr[1][0][c], 0x07060302u),
                           __builtin_amdgcn_perm(vr[1][3][c], vr[1][2][c], 0x07060302u)};
        o[cb][2 * c] = mfma16x16x32<DT>(pa, blo, o[cb][2 * c]);
        o[cb][2 * c + 1] = mfma16x16x32<DT>(pa, bhi, o[cb][2 * c + 1]);
        if constexpr (kSplitP) {
          o[cb][2 * c] = mfma16x16x32<DT>(pl, blo, o[cb][2 * c]);
          o[cb][2 * c + 1] = mfma16x16x32<DT>(pl, bhi, o[cb][2 * c + 1]);
        }
      }
    }

    if (t + 1 < n_tiles) {
      // Every wave finished reading buffer buf^1 before the barrier that ended
      // the previous tile, so it can take tile t+1 now.
      store_tile(buf ^ 1);
    }
    __syncthreads();
  }

  // out[column] = o / l; the column sum of weights lives in lanes i16 = column.
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    float lcol = lsum[cb] + __shfl_xor(lsum[cb], 16);
    lcol += __shfl_xor(lcol, 32);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = 4 * kg + r;
      const float lr = __shfl(lcol, col);
      const int qi = q0 + (wv * CB + cb) * qpb + col / a.n_rep;
      const int hh = g * a.n_rep + col % a.n_rep;
      if (qi < C && hh < a.Hq) {
        float vals[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vals[e] = o[cb][e][r] / lr;
        u32x4 packed;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          packed[c] = uint32_t(Elem<DT>::from_float(vals[2 * c])) | (uint32_t(Elem<DT>::from_float(vals[2 * c + 1])) << 16);
        }
        *reinterpret_cast<u32x4*>(a.out + ((int64_t)(q_begin + qi) * a.Hq + hh) * D + 8 * i16) = packed;
      }
    }
  }
}

// Reference-order scalar prefill for shapes the MFMA kernel does not cover: one
// workgroup per (q head, query row); natural exp; keys 0 .. P + i in page order.
template <int DT>
__global__ void __launch_bounds__(256) paged_prefill_scalar_kernel(const PrefillArgs a) {
  const int row = blockIdx.x;
  const int h = blockIdx.y;
  // sequence of this query row
  int b = 0;
  while (b + 1 < a.B && a.cu_q[b + 1] <= row) ++b;
  const int C = a.cu_q[b + 1] - a.cu_q[b];
  const int i = row - a.cu_q[b];
  if (i < 0 || i >= C) return;
  const int Lk = kv_len_of(a, b);
  const int L = max(0, min(Lk, Lk - C + i + 1));
  const int g = h / a.n_rep;
  const int tid = threadIdx.x, t = tid >> 4, sub = tid & 15;
  __shared__ float qs[256];
  __shared__ float ss[16];
  const uint16_t* qrow = a.q + (int64_t)row * a.q_st + (int64_t)h * a.q_sh;
  for (int d = tid; d < a.D; d += blockDim.x) qs[d] = Elem<DT>::one(qrow[d]);
  __syncthreads();
  const int n_pages = (L + 15) >> 4;
  const int d = tid;
  float m = kNegFltMax, l = 0.f, acc = 0.f;
  for (int pg = 0; pg < n_pages; ++pg) {
    int bid = a.bt[(int64_t)b * a.max_blocks + pg];
    const bool ok = (unsigned)bid < (unsigned)a.num_pages;
    bid = ok ? bid : 0;
    const int nv = ok ? min(16, L - 16 * pg) : 0;
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
  if (d < a.D) a.out[((int64_t)row * a.Hq + h) * a.D + d] = Elem<DT>::from_float(acc / l);
}

// Chunk K/V rows into their pages: row cu_q[b] + i goes to position P_b + i.
struct VarlenWriteArgs {
  uint16_t* k_pool;
  uint16_t* v_pool;
  int64_t k_sp, k_st, k_sh, v_sp, v_st, v_sh;
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t n_st, n_sh;  // [total][H][D] strides shared by k_new and v_new
  const int32_t* bt;
  const int32_t* cu_q;
  const int32_t* kv_lens;
  int B, H, D, max_blocks, num_pages, vec;
};

// grid (token blocks of 16, B): block (tb, b) writes 16 chunk tokens of sequence b.
__global__ void __launch_bounds__(256) kv_write_varlen_kernel(const VarlenWriteArgs a) {
  const int b = blockIdx.y;
  const int q_begin = a.cu_q[b];
  const int C = a.cu_q[b + 1] - q_begin;
  const int cap = a.max_blocks * 16;
  const int Lk = min(max(a.kv_lens[b], 0), cap);
  const int P0 = Lk - C;
  const int per = a.vec ? a.D / 8 : a.D;
  const int items = 16 * a.H * per;
  for (int it = threadIdx.x; it < items; it += blockDim.x) {
    const int c = it % per;
    const int h = (it / per) % a.H;
    const int i = blockIdx.x * 16 + it / (per * a.H);
    if (i >= C) continue;
    const int pos = P0 + i;
    if (pos < 0 || pos >= cap) continue;
    const int page = a.bt[(int64_t)b * a.max_blocks + (pos >> 4)];
    if ((unsigned)page >= (unsigned)a.num_pages) continue;
    const int64_t e = a.vec ? 8 * c : c;
    const int64_t src = (int64_t)(q_begin + i) * a.n_st + (int64_t)h * a.n_sh + e;
    uint16_t* kd = a.k_pool + (int64_t)page * a.k_sp + (int64_t)(pos & 15) * a.k_st + (int64_t)h * a.k_sh + e;
    uint16_t* vd = a.v_pool + (int64_t)page * a.v_sp + (int64_t)(pos & 15) * a.v_st + (int64_t)h * a.v_sh + e;
    if (a.vec) {
      *reinterpret_cast<u32x4*>(kd) = *reinterpret_cast<const u32x4*>(a.k_new + src);
      *reinterpret_cast<u32x4*>(vd) = *reinterpret_cast<const u32x4*>(a.v_new + src);
    } else {
      *kd = a.k_new[src];
      *vd = a.v_new[src];
    }
  }
}

namespace {
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool mul8(int64_t x) { return (x & 7) == 0; }

#ifndef UKV_PREFILL_CB
#define UKV_PREFILL_CB 2
#endif
}  // namespace
}  // namespace ukv

using namespace ukv;

extern "C" int ukv_kv_write_varlen(void* k_pool_layer, void* v_pool_layer, const int64_t* k_strides,
                                   const int64_t* v_strides, const void* k_new, const void* v_new,
                                   const int64_t* new_strides, const int32_t* block_table, int max_blocks,
                                   const int32_t* cu_seqlens_q, const int32_t* kv_lens, int batch, int max_chunk,
                                   int num_heads, int head_dim, int num_pages, ukv_stream_t stream) {
  if (batch < 0 || max_chunk < 0 || num_heads <= 0 || head_dim <= 0 || max_blocks < 0) return UKV_ERR_INVALID_ARGUMENT;
  if (batch == 0 || max_chunk == 0) return UKV_OK;
  if (!k_pool_layer || !v_pool_layer || !k_strides || !v_strides || !k_new || !v_new || !new_strides ||
      !block_table || !cu_seqlens_q || !kv_lens)
    return UKV_ERR_INVALID_ARGUMENT;
  VarlenWriteArgs a{};
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
  a.n_st = new_strides[0];
  a.n_sh = new_strides[1];
  a.bt = block_table;
  a.cu_q = cu_seqlens_q;
  a.kv_lens = kv_lens;
  a.B = batch;
  a.H = num_heads;
  a.D = head_dim;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.vec = head_dim % 8 == 0 && al16(k_pool_layer) && al16(v_pool_layer) && al16(k_new) && al16(v_new) &&
          mul8(a.k_sp) && mul8(a.k_st) && mul8(a.k_sh) && mul8(a.v_sp) && mul8(a.v_st) && mul8(a.v_sh) &&
          mul8(a.n_st) && mul8(a.n_sh);
  const dim3 grid((max_chunk + 15) / 16, batch);
  hipLaunchKernelGGL(kv_write_varlen_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}

extern "C" int ukv_paged_prefill(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                                 const int32_t* cu_seqlens_q, const int32_t* kv_lens, void* out, int batch,
                                 int total_q, int max_chunk, int num_q_heads, int num_kv_heads, int head_dim,
                                 int n_rep, int max_blocks, int num_pages, const int64_t* q_strides,
                                 const int64_t* k_strides, const int64_t* v_strides, float softmax_scale,
                                 int dtype, ukv_stream_t stream_handle) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0) return UKV_ERR_EMPTY;
  if (head_dim > 256) return UKV_ERR_HEAD_DIM;
  if (dtype != UKV_DTYPE_F16 && dtype != UKV_DTYPE_BF16) return UKV_ERR_DTYPE;
  if (num_kv_heads <= 0 || n_rep < 1) return UKV_ERR_GQA;
  const int n_groups = (num_q_heads + n_rep - 1) / n_rep;
  if (n_groups > num_kv_heads) return UKV_ERR_GQA;
  if (total_q < 0 || max_chunk < 0 || max_blocks < 0 || num_pages < 0) return UKV_ERR_INVALID_ARGUMENT;
  if (total_q == 0) return UKV_OK;
  if (!q || !out || !cu_seqlens_q || !kv_lens || !q_strides || !k_strides || !v_strides)
    return UKV_ERR_INVALID_ARGUMENT;
  if (max_blocks > 0 && (!block_table || !k_cache || !v_cache || num_pages <= 0)) return UKV_ERR_INVALID_ARGUMENT;
  PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.out = static_cast<uint16_t*>(out);
  a.k = static_cast<const uint16_t*>(k_cache);
  a.v = static_cast<const uint16_t*>(v_cache);
  a.q_st = q_strides[0];
  a.q_sh = q_strides[1];
  a.k_sp = k_strides[0];
  a.k_st = k_strides[1];
  a.k_sh = k_strides[2];
  a.v_sp = v_strides[0];
  a.v_st = v_strides[1];
  a.v_sh = v_strides[2];
  a.bt = block_table;
  a.cu_q = cu_seqlens_q;
  a.kv_lens = kv_lens;
  a.B = batch;
  a.Hq = num_q_heads;
  a.n_rep = n_rep;
  a.n_groups = n_groups;
  a.D = head_dim;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * kLog2e;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
  const bool strides_ok = mul8(a.q_st) && mul8(a.q_sh) && mul8(a.k_sp) && mul8(a.k_st) && mul8(a.k_sh) &&
                          mul8(a.v_sp) && mul8(a.v_st) && mul8(a.v_sh);
  const bool fast = head_dim == 128 && (n_rep == 1 || n_rep == 2 || n_rep == 4 || n_rep == 8 || n_rep == 16) &&
                    strides_ok && al16(q) && al16(out) && al16(k_cache) && al16(v_cache) && max_blocks > 0;
  if (fast) {
    constexpr int CB = UKV_PREFILL_CB;
    const int qw = 4 * CB * (16 / n_rep);
    const dim3 grid((max_chunk + qw - 1) / qw, n_groups, batch);
    if (dtype == UKV_DTYPE_BF16)
      hipLaunchKernelGGL((paged_prefill_kernel<UKV_DTYPE_BF16, CB>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((paged_prefill_kernel<UKV_DTYPE_F16, CB>), grid, dim3(256), 0, stream, a);
  } else {
    const dim3 grid(total_q, num_q_heads);
    if (dtype == UKV_DTYPE_BF16)
      hipLaunchKernelGGL(paged_prefill_scalar_kernel<UKV_DTYPE_BF16>, grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(paged_prefill_scalar_kernel<UKV_DTYPE_F16>, grid, dim3(256), 0, stream, a);
  }
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}
