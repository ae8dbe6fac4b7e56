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
// Kernel: one workgroup of W waves (W = 8, two per SIMD) takes QW = W * CB *
// (16 / n_rep) consecutive queries of one KV group. Within a wave, an MFMA
// column is a (query, q head) pair: 16 / n_rep queries times the n_rep q heads
// of the group, so one K/V read serves the whole GQA group; a wave holds CB
// 16-column blocks, three or two.
//   * block plan: the chunk of each (sequence, group) is cut from its end down
//     into three-column blocks and then two-column ones (three are cheaper per
//     query, two fill the last round of the launch: the host picks the mix that
//     its model of the dispatch finishes first); each XCD (dispatch is
//     round-robin over the 8 XCDs) runs a contiguous range of (sequence, group)
//     pairs, three-column blocks first: the query blocks of one pair share that
//     XCD's L2 while they stream the same pages;
//   * key tiles of 32 keys (two pages) pass through registers into a 4-slot
//     LDS ring (rows padded to 288 B), written two tiles ahead of their use,
//     with a barrier after every second tile; the loads of tiles t+3 and t+4
//     are in flight while tile t is computed;
//   * S^T = K Q^T on v_mfma_f32_16x16x32 in the input type (A = 16 keys x 32
//     dims from LDS, B = the wave's q columns in registers); lane l ends with
//     keys 4*(l/16) + r of column l % 16;
//   * online softmax per column in log2 units; masks only on tiles that touch
//     the sequence end, an invalid page or the causal diagonal; the running max
//     moves only when a weight reaches 2^8 (wave vote on the packed weights);
//   * P.V on v_mfma_f32_16x16x32_f16: P is rounded to fp16 (11 significant
//     bits, 4x finer than a bf16 P) and, for bf16 pools, the loader converts
//     the V tile to fp16, which is exact for |v| < 65520; a workgroup whose
//     keys hold a larger or non-finite bf16 V recomputes its columns on an
//     fp32 path. The S^T layout is already P's A-operand layout; V's B
//     operands come from ds_read_b64_tr_b16 transpose reads; the softmax
//     denominators come from one more MFMA against a ones operand, so they sum
//     exactly the rounded P;
//   * SnapKV row statistics: the blocks holding each sequence's last obs queries
//     also write those rows' running max and denominator; obs_rows_finish_kernel
//     then sums the sink and window keys' weights again from the same scores and
//     takes them off, leaving the middle keys' sum.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <functional>
#include <map>
#include <mutex>
#include <queue>
#include <tuple>
#include <type_traits>
#include <vector>

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
  // Query blocks of every (sequence, KV group), from the end of its chunk down: n3 blocks of three
  // column blocks per wave, then n2 of two. Blocks that reach below the chunk's first query are
  // partial or empty (chunks shorter than the longest). The three-column blocks of every pair are
  // dispatched in a first pass, the two-column ones in a second.
  int n3, n2;
  // The longest chunk the caller declared: the block plan covers that many queries. A chunk
  // longer than it gets NaN in every row of its output (its K/V were not all written either).
  int max_chunk;
  float scale, scale_log2;
  // SnapKV observation statistics (obs > 0): for each of a sequence's last obs queries and q head
  // h, the log2-sum-exp2 of its scaled scores over the middle keys [sink, L - obs) and the zero
  // rows that pad them to a multiple of 16 keys: obs_stats[b * stats_seq_stride + h * obs + i].x
  // (.y = 0, or 1 where the sum lost precision), the row statistics the SnapKV scoring pass takes.
  // The prefill kernel leaves each row's (max, denominator) there and obs_rows_finish_kernel
  // takes the sink and window keys' share off.
  float2* obs_stats;
  int64_t stats_seq_stride;
  int sink, obs;
};

__device__ __forceinline__ int kv_len_of(const PrefillArgs& a, int b) {
  const int cap = a.max_blocks * 16;
  const int L = a.kv_lens[b];
  return L < 0 ? 0 : (L > cap ? cap : L);
}

// Two bf16 values -> two fp16 values (RNE; exact when 2^-14 <= |x| < 65520). A bf16 value
// that fp16 cannot hold (|x| >= 65536, the next bf16 above 65280; inf; NaN) becomes an fp16
// inf or NaN.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
  return pack_f16(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
}

// Tile loads whose completion the kernel waits for itself. Two register sets
// are in flight while a tile is computed; the compiler's own wait placement
// cannot see which set is older across the unrolled loop and waits for both,
// so the loads are issued here and vm_wait<N>() waits until at most N vector
// memory operations are outstanding. The "+v" operands make every use of the
// loaded registers follow the wait.
__device__ __forceinline__ void gload16(u32x4& r, const void* p) {
  asm volatile("global_load_dwordx4 %0, %1, off" : "=&v"(r) : "v"(p));
}
template <int N> __device__ __forceinline__ void vm_wait(u32x4& x, u32x4& y) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}

// 8-byte LDS transpose read (ds_read_b64_tr_b16).
__device__ __forceinline__ u32x2 ds_read_tr16(const uint16_t* p) {
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

#ifndef UKV_PREFILL_WAVES
#define UKV_PREFILL_WAVES 8
#endif

constexpr int kTileKeys = 32;
// LDS row pitches in 16-bit elements: K and V rows sit 288 B apart, the pitch
// at which SQ_LDS_BANK_CONFLICT reads 0 for the 16-row x 16-byte K reads, the
// 4-row x 32-byte V transpose reads and the 16-byte row stores (272 B leaves
// the K reads conflicting).
#ifndef UKV_PREFILL_KPAD
#define UKV_PREFILL_KPAD 144
#endif
#ifndef UKV_PREFILL_VPAD
#define UKV_PREFILL_VPAD 144
#endif
constexpr int kRowPad = UKV_PREFILL_KPAD;
constexpr int kVRowPad = UKV_PREFILL_VPAD;
constexpr int kStages = 4;  // K/V ring slots: tiles are written two ahead, a barrier every second tile

// Fallback for a workgroup whose key range holds a bf16 V value of magnitude
// >= 65520 (or infinite), which fp16 cannot carry: every (query, head) pair
// of the workgroup is recomputed in fp32 on the vector ALUs, one pair per
// wave at a time, keys in page order (the reference's order), natural exp.
// D = 128: lane l owns dims 2l and 2l + 1.
template <int DT>
__device__ void prefill_pairs_fp32(const PrefillArgs& a, int b, int g, int q_begin, int C, int P0, int Lk, int qa,
                                   int qe, int wv, int nwaves, int lane) {
  const int32_t* btrow = a.bt + (int64_t)b * a.max_blocks;
  const int npairs = (qe - qa) * a.n_rep;
  for (int pi = wv; pi < npairs; pi += nwaves) {
    const int qi = qa + pi / a.n_rep;
    const int h = g * a.n_rep + pi % a.n_rep;
    if (qi >= C || h >= a.Hq) continue;
    const int L = max(0, min(Lk, P0 + qi + 1));
    const uint16_t* qrow = a.q + (int64_t)(q_begin + qi) * a.q_st + (int64_t)h * a.q_sh + 2 * lane;
    const float q0 = Elem<DT>::one(qrow[0]), q1 = Elem<DT>::one(qrow[1]);
    float m = kNegFltMax, l = 0.f, acc0 = 0.f, acc1 = 0.f;
    for (int key = 0; key < L; ++key) {
      const int id = btrow[key >> 4];
      if ((unsigned)id >= (unsigned)a.num_pages) continue;
      const uint16_t* kr = a.k + (int64_t)id * a.k_sp + (int64_t)(key & 15) * a.k_st + (int64_t)g * a.k_sh + 2 * lane;
      const uint16_t* vr = a.v + (int64_t)id * a.v_sp + (int64_t)(key & 15) * a.v_st + (int64_t)g * a.v_sh + 2 * lane;
      float part = q0 * Elem<DT>::one(kr[0]) + q1 * Elem<DT>::one(kr[1]);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
      const float sc = part * a.scale;
      const float mn = fmaxf(m, sc);
      const float alpha = expf(m - mn), pk = expf(sc - mn);
      l = l * alpha + pk;
      acc0 = acc0 * alpha + pk * Elem<DT>::one(vr[0]);
      acc1 = acc1 * alpha + pk * Elem<DT>::one(vr[1]);
      m = mn;
    }
    uint16_t* orow = a.out + ((int64_t)(q_begin + qi) * a.Hq + h) * 128 + 2 * lane;
    orow[0] = Elem<DT>::from_float(acc0 / l);
    orow[1] = Elem<DT>::from_float(acc1 / l);
  }
}

// Flags (y = 1) the observation rows among queries lo .. hi - 1 of sequence b's chunk (C
// queries), q heads of KV group g, for the scoring pass to recompute from the keys.
template <int WAVES>
__device__ void flag_obs_rows(const PrefillArgs& a, int b, int g, int C, int lo, int hi) {
  lo = max(lo, C - a.obs);
  const int n = max(0, min(hi, C) - lo) * a.n_rep;
  for (int t = threadIdx.x; t < n; t += 64 * WAVES) {
    const int qi = lo + t / a.n_rep, h = g * a.n_rep + t % a.n_rep;
    if (qi >= 0 && h < a.Hq)
      a.obs_stats[(int64_t)b * a.stats_seq_stride + (int64_t)h * a.obs + (qi - (C - a.obs))] = make_float2(NAN, 1.f);
  }
}

// LDS of one workgroup: kStages ring slots of K and V (fp16) tiles.
struct PrefillLds {
  __attribute__((aligned(16))) uint16_t k_s[kStages][kTileKeys][kRowPad];
  __attribute__((aligned(16))) uint16_t v_s[kStages][kTileKeys][kVRowPad];
};

// The query block q0 .. q0 + QW - 1 (QW = WAVES * CB * 16 / n_rep; q0 may be negative) of
// sequence b, KV group g, with CB 16-column blocks per wave. With statistics (obs > 0) it also
// writes, for each of the sequence's last obs queries in the block and each q head h, the pair
// (m, l) of the column's running max m (log2 units) and its softmax denominator l (the sum of the
// fp16 weights 2^(s * scale * log2e - m) over every key the query sees) into
// obs_stats[b * stats_seq_stride + h * obs + i], for obs_rows_finish_kernel.
template <int DT, int WAVES, int CB>
__device__ __forceinline__ void prefill_tile(const PrefillArgs& a, const int b, const int g, const int q0,
                                             PrefillLds& lds) {
  constexpr int D = 128;
  constexpr int STEPS = D / 32;
  constexpr int NT = 64 * WAVES;
  constexpr int ITEMS = kTileKeys * 16 / NT;  // 16-byte chunks per thread per tensor per tile
  constexpr float kTau = 8.f;
  constexpr bool kBf16 = DT == UKV_DTYPE_BF16;
  static_assert(ITEMS * NT == kTileKeys * 16, "loader mapping");
  auto& k_s = lds.k_s;
  auto& v_s = lds.v_s;  // fp16

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int i16 = lane & 15;
  const int kg = lane >> 4;

  const int qpb = 16 / a.n_rep;  // queries per column block
  const int qw = WAVES * CB * qpb;
  const int q_begin = a.cu_q[b];
  const int C = a.cu_q[b + 1] - q_begin;
  if (q0 >= C || q0 + qw <= 0) return;  // whole workgroup
  const int Lk = kv_len_of(a, b);
  const int P0 = Lk - C;  // keys before the chunk
  const int kend = max(0, min(Lk, P0 + min(C, q0 + qw)));
  const int n_tiles = (kend + kTileKeys - 1) / kTileKeys;
  const int n_pg = (kend + 15) >> 4;

  // This wave's queries and this lane's columns.
  const int wq0 = q0 + wv * CB * qpb;
  const bool wave_live = wq0 < C && wq0 + CB * qpb > 0;
  const int wpos_min = P0 + wq0;
  const int head = g * a.n_rep + i16 % a.n_rep;
  // the query of this lane's column in column block cb is qi0 + cb * qpb (unused if outside 0 .. C - 1)
  const int qi0 = wq0 + i16 / a.n_rep;
  u32x4 qv[CB][STEPS];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int qi = qi0 + cb * qpb;
    const bool live = qi >= 0 && qi < C && head < a.Hq;
    const uint16_t* qp = a.q + (int64_t)(q_begin + (live ? qi : 0)) * a.q_st + (int64_t)(live ? head : 0) * a.q_sh +
                         8 * kg;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) qv[cb][s] = live ? ld16(qp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
  }

  float m_ref[CB];  // running max of the column (log2 units)
  f32x4 o[CB][8];
  f32x4 lacc[CB];  // softmax denominators of columns 4*kg + r
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    m_ref[cb] = kNegFltMax;
    lacc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 8; ++e) o[cb][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- tile loader: chunk idx = tid + i * NT is 16-byte chunk idx % 16 of key row idx / 16.
  // Tile u is loaded into register set u & 1 four tiles ahead, written into
  // ring slot u % 4 two tiles ahead (zeroing rows past the sequence or on an
  // invalid page and converting a bf16 V to fp16), and computed at tile u.
  // The block table is read through the constant address space: the kernel
  // never writes it, and this keeps the wave-uniform page-id loads on the
  // scalar unit (SMEM), apart from the vector-memory count the tile loads use.
  typedef const __attribute__((address_space(4))) int32_t cint32;
  cint32* btrow = (cint32*)(a.bt + (int64_t)b * a.max_blocks);
  auto page_id = [&](int pg) -> int { return pg < n_pg ? btrow[pg] : -1; };
  auto page_ok = [&](int id) -> bool { return (unsigned)id < (unsigned)a.num_pages; };
  // Within a page, this thread's chunk sits at a fixed offset; the page base is wave-uniform.
  uint32_t koff[ITEMS], voff[ITEMS];
  int lds_row[ITEMS], lds_ch[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int idx = tid + i * NT;
    const int tok = (idx >> 4) & 15, ch = idx & 15;
    koff[i] = (uint32_t)(tok * a.k_st + g * a.k_sh + 8 * ch);
    voff[i] = (uint32_t)(tok * a.v_st + g * a.v_sh + 8 * ch);
    lds_row[i] = idx >> 4;
    lds_ch[i] = ch;
  }
  u32x4 rk0[ITEMS], rv0[ITEMS], rk1[ITEMS], rv1[ITEMS];
  auto issue = [&](int id0, int id1, u32x4 (&rk)[ITEMS], u32x4 (&rv)[ITEMS]) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      // rows 0-15 of a tile come from its first page, rows 16-31 from the second
      const int second = __builtin_amdgcn_readfirstlane((tid + i * NT) >> 8);
      const int id = second ? id1 : id0;
      // page strides fit 32 bits (checked on the host): a 32 x 32 -> 64-bit scalar product
      const uint32_t pg = page_ok(id) ? (uint32_t)id : 0u;
      gload16(rk[i], a.k + (uint64_t)pg * (uint32_t)a.k_sp + koff[i]);
      gload16(rv[i], a.v + (uint64_t)pg * (uint32_t)a.v_sp + voff[i]);
    }
  };
  // The largest and the smallest fp16 V value this thread stored, over every tile (three-input
  // packed maximum / minimum, which carry a NaN through): checked once after the loop for an
  // inf or NaN, i.e. a bf16 value fp16 cannot hold.
  typedef _Float16 hv2 __attribute__((ext_vector_type(2)));
  hv2 vmax = {0, 0}, vmin = {0, 0};
  auto store = [&](int u, int slot, int id0, int id1, u32x4 (&rk)[ITEMS], u32x4 (&rv)[ITEMS]) {
    const bool full = page_ok(id0) && page_ok(id1) && kTileKeys * (u + 1) <= Lk;
    // The other register set's 2 * ITEMS loads were issued after this set's.
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) vm_wait<2 * ITEMS>(rk[i], rv[i]);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      // (converted before the junk rows are zeroed: the conversion writes new registers, which
      // the zeroing then selects in place, with no copy of the loaded ones)
      u32x4 v;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = kBf16 ? bf16x2_to_f16x2(rv[i][c]) : rv[i][c];
      if (!full) {  // (wave-uniform) rows past the sequence or on an invalid page hold junk
        const bool ok = page_ok(lds_row[i] < 16 ? id0 : id1) && kTileKeys * u + lds_row[i] < Lk;
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = ok ? v[c] : 0u;
      }
      if constexpr (kBf16) {
        const uint32_t w0 = v[0], w1 = v[1], w2 = v[2], w3 = v[3];
        const hv2 c0 = __builtin_bit_cast(hv2, w0), c1 = __builtin_bit_cast(hv2, w1);
        const hv2 c2 = __builtin_bit_cast(hv2, w2), c3 = __builtin_bit_cast(hv2, w3);
        vmax = __builtin_elementwise_maximum(__builtin_elementwise_maximum(vmax, c0), c1);
        vmax = __builtin_elementwise_maximum(__builtin_elementwise_maximum(vmax, c2), c3);
        vmin = __builtin_elementwise_minimum(__builtin_elementwise_minimum(vmin, c0), c1);
        vmin = __builtin_elementwise_minimum(__builtin_elementwise_minimum(vmin, c2), c3);
      }
      *reinterpret_cast<u32x4*>(&k_s[slot][lds_row[i]][8 * lds_ch[i]]) = rk[i];
      *reinterpret_cast<u32x4*>(&v_s[slot][lds_row[i]][8 * lds_ch[i]]) = v;
    }
  };

  // Page ids of tiles t .. t+3 (t_id[j] = tile t + j).
  int t_id[4][2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t_id[j][0] = page_id(2 * j);
    t_id[j][1] = page_id(2 * j + 1);
  }
  // Prologue: tiles 0 and 1 into the ring, tiles 2 and 3 in flight. Loads are issued
  // unconditionally (tiles past the end read page 0 and are never used) so
  // that every wait is on loads of a fixed age: vmcnt(2) on the older set.
  issue(t_id[0][0], t_id[0][1], rk0, rv0);
  issue(t_id[1][0], t_id[1][1], rk1, rv1);
  store(0, 0, t_id[0][0], t_id[0][1], rk0, rv0);
  issue(t_id[2][0], t_id[2][1], rk0, rv0);
  store(1, 1, t_id[1][0], t_id[1][1], rk1, rv1);
  issue(t_id[3][0], t_id[3][1], rk1, rv1);
  int id_n0 = page_id(8), id_n1 = page_id(9);  // page ids of tile t+4
  // Retire every load issued so far (q columns, tiles 2 and 3) once, so that
  // no wait for them is left inside the loop.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();

  // Tiles t < n_full end below the sequence end and below every column's diagonal (key
  // 32t + 31 <= min(Lk - 1, wpos_min)).
  const int n_full = max(0, min(Lk, wpos_min + 1)) / kTileKeys;
  const float sl2 = a.scale_log2;
  const uint32_t ones_f16 = 0x3C003C00u;

  auto compute = [&](int t, int slot) {
    const int key0 = t * kTileKeys;
    const bool pg0 = page_ok(t_id[0][0]), pg1 = page_ok(t_id[0][1]);
    const bool full = pg0 && pg1 && t < n_full;
    // S^T[key][column] for the tile's two 16-key blocks and every column block, masked. (As one
    // inlined function the register allocator keeps the three-column loop within 256 VGPRs with
    // no scratch under the iterative-ILP schedule this file is built with; written out in line,
    // that schedule needed 20 bytes per lane of scratch.)
    auto scores = [&](f32x4 (&sacc)[2][CB]) __attribute__((always_inline)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) sacc[kb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
          const u32x4 ka = *reinterpret_cast<const u32x4*>(&k_s[slot][kb * 16 + i16][32 * s + 8 * kg]);
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) sacc[kb][cb] = mfma16x16x32<DT>(ka, qv[cb][s], sacc[kb][cb]);
        }
      }
      if (!full) {
        // key kb*16 + 4kg + r is visible to a column iff it is below lim[kb]
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const int qi = qi0 + cb * qpb;
          const bool live = qi >= 0 && qi < C && head < a.Hq;
          const int vis = live ? min(Lk, P0 + qi + 1) - key0 - 4 * kg : -1;  // an unused column sees no key
          const int lim0 = pg0 ? vis : 0, lim1 = pg1 ? vis - 16 : 0;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) sacc[kb][cb][r] = r < (kb ? lim1 : lim0) ? sacc[kb][cb][r] : -INFINITY;
        }
      }
    };
    f32x4 sacc[2][CB];
    scores(sacc);
    // Softmax: p = 2^(s*scale*log2e - m) as fp16 against the running max m
    // (log2 units) of its column. m moves only when some p of the tile reaches
    // 2^8: the packed fp16 P is checked (non-negative fp16 bit patterns order
    // like their values, and inf and NaN lie above), and a column block whose
    // max moved is rescaled and its P recomputed.
    u32x4 pa[CB];
    auto exp_pack = [&](int cb) {
      float p[2][4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) p[kb][r] = fast_exp2(__builtin_fmaf(sacc[kb][cb][r], sl2, -m_ref[cb]));
      pa[cb] = u32x4{pack_f16(p[0][0], p[0][1]), pack_f16(p[0][2], p[0][3]), pack_f16(p[1][0], p[1][1]),
                     pack_f16(p[1][2], p[1][3])};
    };
    // Moves column block cb's max to the tile's where that lies more than kTau above it,
    // rescaling what was summed under the old one; returns whether it moved.
    auto settle = [&](int cb) -> bool {
      float mloc = sacc[0][cb][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, sacc[kb][cb][r]);
      float mcol = fmaxf(mloc, __shfl_xor(mloc, 16));
      mcol = fmaxf(mcol, __shfl_xor(mcol, 32));
      if (!__any(mcol * sl2 > m_ref[cb] + kTau)) return false;
      const float m_new = fmaxf(m_ref[cb], mcol * sl2);
      const float alpha = fast_exp2(m_ref[cb] - m_new);
      m_ref[cb] = m_new;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * kg + r);
        lacc[cb][r] *= ar;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[cb][e][r] *= ar;
      }
      return true;
    };
    // The weights and the vote run at raised wave priority: when the SIMD's other wave is
    // issuing its MFMAs, this wave's softmax VALU work goes first (4-5 % faster at config 4
    // than without; raising it from the mask check on, to priority 3, or for the loader's
    // stores as well measured slower).
    __builtin_amdgcn_s_setprio(1);
    {  // the tile's weights, then the vote on them
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) exp_pack(cb);
      // The max of the packed weights with three-input fp16 maxima (v_pk_maximum3_f16): a NaN
      // weight makes the maximum NaN, whose pattern, like inf's, lies above the threshold.
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      // (the element is copied out first: clang lowers __builtin_bit_cast of a vector element
      // lvalue to a load of the vector's first element, whatever the index)
      auto hv = [&](int i) {
        const uint32_t w = pa[i / 4][i % 4];
        return __builtin_bit_cast(h2, w);
      };
      h2 mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(hv(0), hv(1)), hv(2));
#pragma unroll
      for (int i = 3; i + 1 < 4 * CB; i += 2)
        mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx, hv(i)), hv(i + 1));
      if constexpr ((4 * CB - 3) % 2) mx = __builtin_elementwise_maximum(mx, hv(4 * CB - 1));
      const u16x2 pmax = __builtin_bit_cast(u16x2, mx);
      if (__any(__builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(pmax, u16x2{0x5BFF, 0x5BFF})) != 0u)) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          if (settle(cb)) exp_pack(cb);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // P.V: the B operand of output tile e (dims 16e .. 16e + 15) holds, in lane
    // (i16, kg), dim 16e + i16 of keys 4kg..4kg+3 and 16+4kg..16+4kg+3 (the
    // key order of P's A operand). ds_read_b64_tr_b16 builds it from row-major
    // V: within each 16-lane group, lane L names 4 dims 4(L%4).. of key row
    // L/4, and lane j receives dim j of the 4 rows.
    const uint16_t* vlane = &v_s[slot][4 * kg + (i16 >> 2)][4 * (i16 & 3)];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const u32x2 lo = ds_read_tr16(vlane + 16 * e);
      const u32x2 hi = ds_read_tr16(vlane + 16 * kVRowPad + 16 * e);
      const u32x4 bv = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) o[cb][e] = mfma16x16x32<UKV_DTYPE_F16>(pa[cb], bv, o[cb][e]);
    }
    // Denominators: the same P against a ones operand.
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
      lacc[cb] = mfma16x16x32<UKV_DTYPE_F16>(pa[cb], u32x4{ones_f16, ones_f16, ones_f16, ones_f16}, lacc[cb]);
  };

  // Tile t: (a) tile t+2 from register set t&1 into ring slot (t+2)%4; (b) tile t+4 into that
  // set; (c) tile t on this wave's columns; (d) after an odd t, a barrier. A slot written at
  // step t is read at step t+2 and written again at step t+4: a barrier after every odd step
  // lies between each write and its reads, and between each read and the next write. The loop
  // is unrolled by the ring's four slots, so slots and register sets are compile-time constants
  // (LDS offsets fold into the instructions; register sets never meet at a runtime join).
  auto step = [&](int t, auto phase, auto do_compute) {
    constexpr int Q = decltype(phase)::value;  // t % 4: the ring slot of tile t
    constexpr int P = Q & 1;                   // register set of tile t+2
    // (a slot written past the last tile is never read)
    if constexpr (P == 0) store(t + 2, (Q + 2) & 3, t_id[2][0], t_id[2][1], rk0, rv0);
    else store(t + 2, (Q + 2) & 3, t_id[2][0], t_id[2][1], rk1, rv1);
    if constexpr (P == 0) issue(id_n0, id_n1, rk0, rv0);
    else issue(id_n0, id_n1, rk1, rv1);
    do_compute(t, Q);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      t_id[j][0] = t_id[j + 1][0];
      t_id[j][1] = t_id[j + 1][1];
    }
    t_id[3][0] = id_n0;
    t_id[3][1] = id_n1;
    id_n0 = page_id(2 * (t + 5));
    id_n1 = page_id(2 * (t + 5) + 1);
    if constexpr (P == 1) __syncthreads();
  };
  auto run = [&](auto do_compute) {
    for (int t = 0; t < n_tiles; t += 4) {
      step(t, std::integral_constant<int, 0>{}, do_compute);
      if (t + 1 < n_tiles) step(t + 1, std::integral_constant<int, 1>{}, do_compute);
      if (t + 2 < n_tiles) step(t + 2, std::integral_constant<int, 2>{}, do_compute);
      if (t + 3 < n_tiles) step(t + 3, std::integral_constant<int, 3>{}, do_compute);
    }
  };
  if (wave_live) run(compute);
  else run([](int, int) {});
  // Loads of tiles past the end are still in flight: retire them while their
  // registers are still held, so that nothing else is placed in them first.
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    vm_wait<0>(rk0[i], rv0[i]);
    vm_wait<0>(rk1[i], rv1[i]);
  }

  // A bf16 V value that fp16 cannot hold anywhere in this workgroup's keys:
  // recompute its columns on the fp32 fallback.
  // (an fp16 magnitude pattern above 0x7BFF, the largest finite one, is an inf or a NaN)
  const u16x2 mag = __builtin_elementwise_max(as_u16x2(__builtin_bit_cast(uint32_t, vmax) & 0x7fff7fffu),
                                              as_u16x2(__builtin_bit_cast(uint32_t, vmin) & 0x7fff7fffu));
  const bool wide_mine = kBf16 && __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(mag, u16x2{0x7BFF, 0x7BFF})) != 0u;
  if (kBf16 && __syncthreads_or(wide_mine)) {
    flag_obs_rows<WAVES>(a, b, g, C, max(q0, 0), min(C, q0 + qw));  // (none without statistics)
    prefill_pairs_fp32<DT>(a, b, g, q_begin, C, P0, Lk, max(q0, 0), min(C, q0 + qw), wv, WAVES, lane);
    return;
  }

  // out[column] = o / l: lane (i16, kg) holds dims 16e + i16 of columns 4*kg + r,
  // and lacc[cb][r] is the denominator of column 4*kg + r (the same in its 16 lanes).
  if (!wave_live) return;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = 4 * kg + r;
      const int qi = wq0 + cb * qpb + col / a.n_rep;
      const int hh = g * a.n_rep + col % a.n_rep;
      // the column's running max, held by lane col (column i16 = col)
      const float m_col = __shfl(m_ref[cb], col);
      if (qi >= 0 && qi < C && hh < a.Hq) {
        const float inv = 1.f / lacc[cb][r];
        uint16_t* orow = a.out + ((int64_t)(q_begin + qi) * a.Hq + hh) * D + i16;
#pragma unroll
        for (int e = 0; e < 8; ++e) orow[16 * e] = Elem<DT>::from_float(o[cb][e][r] * inv);
        if (i16 == 0 && qi >= C - a.obs)  // (never without statistics: obs = 0)
          a.obs_stats[(int64_t)b * a.stats_seq_stride + (int64_t)hh * a.obs + (qi - (C - a.obs))] =
              make_float2(m_col, lacc[cb][r]);
      }
    }
  }
}

// Rows lo .. hi - 1 of sequence b's chunk, the q heads of KV group g, set to NaN (0x7FFF is a
// NaN in fp16 and in bf16). For chunks longer than the declared max_chunk: the block plan does not
// reach their first queries and the chunk write stopped at max_chunk tokens, so every block of
// such a chunk writes NaN into its rows instead of attending, the lowest block also into the rows
// below it.
template <int WAVES>
__device__ void prefill_nan_rows(const PrefillArgs& a, int b, int g, int lo, int hi) {
  const int h0 = g * a.n_rep;
  const int per = min(a.n_rep, a.Hq - h0) * a.D;  // a query row's heads of the group, contiguous
  const int64_t n = (int64_t)max(0, hi - lo) * per;
  uint16_t* base = a.out + ((int64_t)(a.cu_q[b] + lo) * a.Hq + h0) * a.D;
  for (int64_t i = threadIdx.x; i < n; i += 64 * WAVES)
    base[(i / per) * a.Hq * a.D + i % per] = 0x7FFFu;
}

// The s-th work item an XCD dispatches from its range [start, end) of pair-major item numbers
// (item j of pair p is number p * n + j): first the items j < nl of the range's pairs, pair by
// pair, then the items j >= nl. Returns false past the range.
__device__ __forceinline__ bool locate_item(int start, int end, int n, int nl, int s, int& pair, int& j) {
  const int p0 = start / n, p1 = (end - 1) / n;
  for (int pass = 0; pass < 2; ++pass) {
    const int lo = pass ? nl : 0, hi = pass ? n : nl, w = hi - lo;  // the pass's item numbers in a pair
    const int c0 = max(0, min(hi, end - p0 * n) - max(lo, start - p0 * n));  // first pair, cut by start
    if (s < c0) {
      pair = p0;
      j = max(lo, start - p0 * n) + s;
      return true;
    }
    s -= c0;
    if (p1 == p0) continue;
    const int whole = max(0, p1 - p0 - 1);  // pairs wholly in the range
    if (s < whole * w) {
      pair = p0 + 1 + s / w;
      j = lo + s % w;
      return true;
    }
    s -= whole * w;
    const int c1 = max(0, min(hi, end - p1 * n) - lo);  // last pair, cut by end
    if (s < c1) {
      pair = p1;
      j = lo + s;
      return true;
    }
    s -= c1;
  }
  return false;
}

// The range of work items [start, end) of a launch's n_items items that XCD xcd runs: dispatch
// is round-robin over the 8 XCDs, so the workgroups with blockIdx.x % 8 == xcd run there, and
// each XCD takes a contiguous range of the item numbers.
__device__ __forceinline__ void xcd_range(int total, int xcd, int& start, int& end) {
  const int per = total >> 3, rem = total & 7;
  start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
  end = start + per + (xcd < rem ? 1 : 0);
}

// Work items: the n3 + n2 query blocks of each (sequence, KV group) ("pair"), numbered pair
// after pair. Each XCD takes a contiguous range of these numbers, so that the blocks of one pair
// share that XCD's L2 while they stream its pages, and dispatches the three-column blocks of its
// pairs before their two-column blocks: the cheaper blocks then fill the last round of the launch.
// With statistics (obs > 0) the blocks also write the (m, l) pairs of the chunk's last obs queries
// (prefill_tile), which obs_rows_finish_kernel turns into SnapKV row statistics. (Launches without
// statistics run the same instance: compiled with that epilogue, the tile loop's schedule is 0.7 %
// faster at config 4 than without it.)
template <int DT, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2)))
paged_prefill_kernel(const PrefillArgs a) {
  __shared__ PrefillLds lds;
  const int n_items = a.n3 + a.n2;
  int start, end, pair, j;
  xcd_range(n_items * a.n_groups * a.B, blockIdx.x & 7, start, end);
  if (!locate_item(start, end, n_items, a.n3, blockIdx.x >> 3, pair, j)) return;  // (never: the grid holds total)
  const int g = pair % a.n_groups, b = pair / a.n_groups;
  const int C = a.cu_q[b + 1] - a.cu_q[b];
  const int qpb = 16 / a.n_rep;
  const int qw2 = WAVES * 2 * qpb, qw3 = WAVES * 3 * qpb;
  if (C > a.max_chunk) {
    const int q0 = j < a.n3 ? C - qw3 * (j + 1) : C - qw3 * a.n3 - qw2 * (j - a.n3 + 1);
    const int q1 = min(C, j < a.n3 ? q0 + qw3 : q0 + qw2);
    const int lo = j == n_items - 1 ? 0 : max(0, q0);
    prefill_nan_rows<WAVES>(a, b, g, lo, q1);
    flag_obs_rows<WAVES>(a, b, g, C, lo, q1);  // (none without statistics)
    return;
  }
  if (j < a.n3)
    prefill_tile<DT, WAVES, 3>(a, b, g, C - qw3 * (j + 1), lds);
  else
    prefill_tile<DT, WAVES, 2>(a, b, g, C - qw3 * a.n3 - qw2 * (j - a.n3 + 1), lds);
}

// SnapKV row statistics from the (m, l) pairs paged_prefill_kernel left in obs_stats.
// l sums the weights 2^(s * scale * log2e - m) of every key the query sees, each rounded to fp16;
// the sink keys [0, sink) and the window keys [max(L - obs, sink), the query's own position] are
// summed again here from the same scores (v_mfma_f32_16x16x32 on the same operands, in the same
// order), exp2 and fp16 rounding, and taken off, which leaves the middle keys [sink, L - obs).
// Where the prefill computed those weights against the final m (m moves only when a weight would
// reach 2^8), they cancel exactly and the sum carries only the middle weights' own fp16 rounding;
// weights taken before a later move of m were rescaled in fp32 and leave a residue of at most
// 2^-11 of their share. The row becomes (log2 of that sum and of
// the zero rows padding the middle keys to a multiple of 16, 0) in the units of s * scale * log2e;
// it is flagged (y = 1) for the scoring pass to recompute from the keys where the prefill flagged
// it, where the sink and window hold half of its weight or more (the difference would lose bits),
// or where the middle sum falls below 2^-100 of its max (m is the max over every key the query
// sees: middle weights below 2^-126 of it lose bits). One wave per 16 columns (observation query,
// q head of the group) of a (sequence, KV group); lane (i16, kg) holds column i16 and keys
// 4kg .. 4kg + 3 of each 16-key page. (The (m, l) pairs exist only where the tiled kernel ran.)
template <int DT>
__global__ void __launch_bounds__(256) obs_rows_finish_kernel(const PrefillArgs a) {
  const int lane = threadIdx.x & 63, i16 = lane & 15, kg = lane >> 4;
  const int cols = a.obs * a.n_rep;
  const int nblk = (cols + 15) >> 4;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (int64_t)a.B * a.n_groups * nblk) return;  // (wave-uniform)
  const int blk = (int)(w % nblk);
  const int64_t pair = w / nblk;
  const int g = (int)(pair % a.n_groups), b = (int)(pair / a.n_groups);
  const int q_begin = a.cu_q[b], C = a.cu_q[b + 1] - q_begin;
  const int L = kv_len_of(a, b);
  const int col = blk * 16 + i16;
  const int i = col / a.n_rep, h = g * a.n_rep + col % a.n_rep;
  const int qi = C - a.obs + i;
  const bool live = col < cols && h < a.Hq && qi >= 0 && C <= a.max_chunk;
  if (!__any(live)) return;  // (wave-uniform: a chunk shorter than the window, or too long)
  float2* slot = a.obs_stats + (int64_t)b * a.stats_seq_stride + (int64_t)h * a.obs + i;
  const float2 ml = live ? *slot : make_float2(0.f, 0.f);
  const bool ok = live && __builtin_isfinite(ml.x) && ml.y > 0.f && __builtin_isfinite(ml.y);
  const float m = ok ? ml.x : 0.f;
  // B operand: dims 32s + 8kg .. 32s + 8kg + 7 of column i16's query row
  const uint16_t* qp = a.q + (live ? (int64_t)(q_begin + qi) * a.q_st + (int64_t)h * a.q_sh : 0) + 8 * kg;
  u32x4 qv[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qv[s] = live ? ld16(qp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
  const int pos = L - C + qi;  // the query's position: it sees keys 0 .. pos
  const float sl2 = a.scale_log2;
  const int32_t* btrow = a.bt + (int64_t)b * a.max_blocks;
  float part = 0.f;
  // Keys [lo, hi) of pages p0 .. p1 - 1 (page pg holds keys 16 pg .. 16 pg + 15), four pages at a
  // time with their loads issued together. A operand: dims 32s + 8kg .. of key 16 pg + i16.
  auto pages = [&](int p0, int p1, int lo, int hi) {
    for (int pg = p0; pg < p1; pg += 4) {
      u32x4 ka[4][4];
      bool pok[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int id = pg + u < p1 ? btrow[pg + u] : -1;
        pok[u] = (unsigned)id < (unsigned)a.num_pages;
        const uint16_t* kp =
            a.k + (int64_t)(pok[u] ? id : 0) * a.k_sp + (int64_t)i16 * a.k_st + (int64_t)g * a.k_sh + 8 * kg;
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[u][s] = pok[u] ? ld16(kp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = mfma16x16x32<DT>(ka[u][s], qv[s], acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = 16 * (pg + u) + 4 * kg + r;
          // the weight rounded to fp16 as the prefill kernel summed it (see above)
          const float p = (float)(_Float16)fast_exp2(__builtin_fmaf(acc[r], sl2, -m));
          part += (pok[u] && key >= lo && key < hi && key <= pos) ? p : 0.f;
        }
      }
    }
  };
  const int s_end = min(a.sink, L), w_beg = max(L - a.obs, a.sink);
  pages(0, (s_end + 15) >> 4, 0, s_end);
  pages(w_beg >> 4, (L + 15) >> 4, w_beg, L);
  part += __shfl_xor(part, 16);
  part += __shfl_xor(part, 32);
  if (kg == 0 && live) {
    float2 res = make_float2(0.f, 1.f);
    if (ok) {
      const float l = ml.y - part;
      const int L_mid = L - a.sink - a.obs;
      const int n_pad = ((L_mid + 15) & ~15) - L_mid;
      const float top = n_pad > 0 ? fmaxf(m, 0.f) : m;
      const float lse = top + __log2f(l * exp2f(m - top) + (float)n_pad * exp2f(-top));
      if (l >= 0.5f * ml.y && l >= 0x1p-100f && __builtin_isfinite(lse)) res = make_float2(lse, 0.f);
    }
    *slot = res;
  }
}

// Marks every observation row of the call as recomputed-by-the-scorer: (0, 1) at row
// obs_stats[b * stats_seq_stride + h * obs + i] for b < B, h < Hq, i < obs.
__global__ void __launch_bounds__(256) obs_flag_kernel(const PrefillArgs a, const int64_t rows) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows) return;
  const int64_t per = (int64_t)a.Hq * a.obs;
  a.obs_stats[(idx / per) * a.stats_seq_stride + idx % per] = make_float2(0.f, 1.f);
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
  if (C > a.max_chunk) {  // longer than declared: its K/V were not all written (see prefill_nan_rows)
    for (int d = threadIdx.x; d < a.D; d += blockDim.x) a.out[((int64_t)row * a.Hq + h) * a.D + d] = 0x7FFFu;
    return;
  }
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
  int per_shift, h_shift;  // log2(D / 8), log2(H) for the 16-byte path (-1: not powers of two)
};

// 16-byte path for power-of-two heads and D / 8: block (tb, b) writes 16 chunk tokens of
// sequence b; 16-byte chunk `it` = (token, head, chunk) by shifts. The two pages the 16
// positions can touch are read once; each pass issues 8 K and 8 V loads before its stores.
__global__ void __launch_bounds__(256) kv_write_varlen_vec_kernel(const VarlenWriteArgs a) {
  constexpr int J = 8;
  const int b = blockIdx.y;
  const int q_begin = a.cu_q[b];
  const int C = a.cu_q[b + 1] - q_begin;
  const int i0 = blockIdx.x * 16;
  if (i0 >= C) return;
  const int cap = a.max_blocks * 16;
  const int Lk = min(max(a.kv_lens[b], 0), cap);
  const int P0 = Lk - C;
  const int blk0 = (P0 + i0) >> 4;  // first page index these 16 positions touch (P0 + i0 >= 0 when valid)
  const int32_t* btrow = a.bt + (int64_t)b * a.max_blocks;
  const int pg0 = (blk0 >= 0 && blk0 < a.max_blocks) ? btrow[blk0] : -1;
  const int pg1 = (blk0 + 1 >= 0 && blk0 + 1 < a.max_blocks) ? btrow[blk0 + 1] : -1;
  const int per_mask = (1 << a.per_shift) - 1, h_mask = (1 << a.h_shift) - 1;
  const int items = 16 << (a.per_shift + a.h_shift);
  for (int base = 0; base < items; base += J * 256) {
    u32x4 kx[J], vx[J];
    uint16_t* kd[J];
    uint16_t* vd[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int it = base + j * 256 + threadIdx.x;
      const int c = it & per_mask;
      const int h = (it >> a.per_shift) & h_mask;
      const int i = i0 + (it >> (a.per_shift + a.h_shift));
      const int pos = P0 + i;
      const int page = ((pos >> 4) == blk0) ? pg0 : pg1;
      const bool ok = it < items && i < C && pos >= 0 && pos < cap && (unsigned)page < (unsigned)a.num_pages;
      kd[j] = ok ? a.k_pool + (int64_t)page * a.k_sp + (int64_t)(pos & 15) * a.k_st + (int64_t)h * a.k_sh + 8 * c
                 : nullptr;
      vd[j] = ok ? a.v_pool + (int64_t)page * a.v_sp + (int64_t)(pos & 15) * a.v_st + (int64_t)h * a.v_sh + 8 * c
                 : nullptr;
      const int64_t src = (int64_t)(q_begin + (ok ? i : i0)) * a.n_st + (int64_t)h * a.n_sh + 8 * c;
      kx[j] = ok ? *reinterpret_cast<const u32x4*>(a.k_new + src) : u32x4{0u, 0u, 0u, 0u};
      vx[j] = ok ? *reinterpret_cast<const u32x4*>(a.v_new + src) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (kd[j]) {
        *reinterpret_cast<u32x4*>(kd[j]) = kx[j];
        *reinterpret_cast<u32x4*>(vd[j]) = vx[j];
      }
    }
  }
}

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
  auto log2_exact = [](int x) {
    int s = 0;
    while ((1 << s) < x) ++s;
    return (1 << s) == x ? s : -1;
  };
  a.per_shift = a.vec ? log2_exact(head_dim / 8) : -1;
  a.h_shift = log2_exact(num_heads);
  const dim3 grid((max_chunk + 15) / 16, batch);
  if (a.vec && a.per_shift >= 0 && a.h_shift >= 0)
    hipLaunchKernelGGL(kv_write_varlen_vec_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(kv_write_varlen_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}

namespace {

// Block plan of the tiled prefill: the numbers n3 and n2 of three- and two-column query blocks
// per (sequence, KV group) that cover its chunk's max_chunk queries. A launch runs in rounds of
// one block per CU; the plan with the shortest predicted launch is taken, modelling every block as streaming equally many keys (a long prefix) at its
// measured cost relative to a three-column block (two columns 0.79: single blocks timed over the
// same 32768 keys), and each XCD's CUs as taking the XCD's blocks in the kernel's order, each CU
// the next block once free.
struct BlockPlan {
  int n3, n2;
};

double plan_makespan(int64_t pairs, int n3, int n2, int cus_per_xcd) {
  const int n_items = n3 + n2;
  const int64_t total = pairs * n_items;
  const int64_t per = total / 8, rem = total % 8;
  double worst = 0.0;
  std::vector<double> order;
  for (int x = 0; x < 8; ++x) {
    const int64_t start = x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
    const int64_t end = start + per + (x < rem ? 1 : 0);
    order.clear();
    if (end > start)
      for (int pass = 0; pass < 2; ++pass)
        for (int64_t p = start / n_items; p <= (end - 1) / n_items; ++p) {
          const int64_t j0 = std::max<int64_t>(pass ? n3 : 0, start - p * n_items);
          const int64_t j1 = std::min<int64_t>(pass ? n_items : n3, end - p * n_items);
          for (int64_t j = j0; j < j1; ++j) order.push_back(j < n3 ? 1.0 : 0.79);
        }
    std::priority_queue<double, std::vector<double>, std::greater<double>> cu;
    for (int c = 0; c < cus_per_xcd; ++c) cu.push(0.0);
    double last = 0.0;
    for (double c : order) {
      const double t = cu.top() + c;
      cu.pop();
      cu.push(t);
      last = std::max(last, t);
    }
    worst = std::max(worst, last);
  }
  return worst;
}

BlockPlan choose_plan(int max_chunk, int64_t pairs, int qw2, int qw3, int cus_per_xcd) {
  const int n3_max = (std::max(0, max_chunk) + qw3 - 1) / qw3;
  BlockPlan best{n3_max, 0};
  // Large launches run many rounds, where the last one matters little: keep three-column blocks.
  if (pairs * n3_max > (1 << 16) || cus_per_xcd <= 0 || n3_max == 0) return best;
  static std::mutex mu;
  static std::map<std::tuple<int, int64_t, int, int>, BlockPlan> cache;
  const auto key = std::make_tuple(max_chunk, pairs, qw2, cus_per_xcd);
  std::lock_guard<std::mutex> lock(mu);
  const auto hit = cache.find(key);
  if (hit != cache.end()) return hit->second;
  double best_t = plan_makespan(pairs, n3_max, 0, cus_per_xcd);
  // Each three-column block traded for two-column ones adds work (0.79 x 1.5 > 1): a dozen
  // trades fill any last round.
  for (int n3 = n3_max - 1; n3 >= std::max(0, n3_max - 12); --n3) {
    const int n2 = (max_chunk - n3 * qw3 + qw2 - 1) / qw2;
    const double t = plan_makespan(pairs, n3, n2, cus_per_xcd);
    if (t < best_t - 1e-9) {
      best_t = t;
      best = BlockPlan{n3, n2};
    }
  }
  if (cache.size() >= 4096) cache.clear();  // a caller cycling through many shapes recomputes
  cache.emplace(key, best);
  return best;
}

// CUs per XCD of the current device (8 XCDs), 0 when unknown.
int cus_per_xcd() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int per = cached[dev].load(std::memory_order_relaxed);
  if (per == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    per = n / 8;
    cached[dev].store(per, std::memory_order_relaxed);
  }
  return per;
}

struct ObsStats {
  void* stats;
  int64_t seq_stride;
  int sink, obs;
};

int prefill_impl(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                 const int32_t* cu_seqlens_q, const int32_t* kv_lens, void* out, int batch, int total_q, int max_chunk,
                 int num_q_heads, int num_kv_heads, int head_dim, int n_rep, int max_blocks, int num_pages,
                 const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides, float softmax_scale,
                 int dtype, ukv_stream_t stream_handle, const ObsStats* obs) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0) return UKV_ERR_EMPTY;
  if (head_dim > 256) return UKV_ERR_HEAD_DIM;
  if (dtype != UKV_DTYPE_F16 && dtype != UKV_DTYPE_BF16) return UKV_ERR_DTYPE;
  if (num_kv_heads <= 0 || n_rep < 1) return UKV_ERR_GQA;
  const int n_groups = (num_q_heads + n_rep - 1) / n_rep;
  if (n_groups > num_kv_heads) return UKV_ERR_GQA;
  if (total_q < 0 || max_chunk < 0 || max_blocks < 0 || num_pages < 0) return UKV_ERR_INVALID_ARGUMENT;
  if (total_q == 0) return UKV_OK;
  // The chunks hold total_q queries, so the longest holds at least total_q / batch of them.
  if ((int64_t)max_chunk * batch < total_q) return UKV_ERR_INVALID_ARGUMENT;
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
  a.max_chunk = max_chunk;
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * kLog2e;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
  // The tiled kernel keeps a row's offset within its page in 32 bits.
  auto in_page_ok = [&](int64_t st, int64_t sh) {
    return st >= 0 && sh >= 0 && 15 * st + (int64_t)(num_kv_heads - 1) * sh + head_dim <= (int64_t)UINT32_MAX;
  };
  auto page_stride_ok = [](int64_t sp) { return sp >= 0 && sp <= (int64_t)UINT32_MAX; };
  const bool strides_ok = mul8(a.q_st) && mul8(a.q_sh) && mul8(a.k_sp) && mul8(a.k_st) && mul8(a.k_sh) &&
                          mul8(a.v_sp) && mul8(a.v_st) && mul8(a.v_sh) && in_page_ok(a.k_st, a.k_sh) &&
                          in_page_ok(a.v_st, a.v_sh) && page_stride_ok(a.k_sp) && page_stride_ok(a.v_sp);
  const bool fast = head_dim == 128 && softmax_scale > 0.f && std::isfinite(softmax_scale) && (n_rep == 1 || n_rep == 2 || n_rep == 4 || n_rep == 8 || n_rep == 16) &&
                    strides_ok && al16(q) && al16(out) && al16(k_cache) && al16(v_cache) && max_blocks > 0;
  if (obs) {
    a.obs_stats = static_cast<float2*>(obs->stats);
    a.stats_seq_stride = obs->seq_stride;
    a.sink = obs->sink;
    a.obs = obs->obs;
  }
  if (fast) {
    constexpr int W = UKV_PREFILL_WAVES;
    const int qw2 = W * 2 * (16 / n_rep), qw3 = W * 3 * (16 / n_rep);
    const int64_t pairs = (int64_t)n_groups * batch;
    const BlockPlan plan = choose_plan(max_chunk, pairs, qw2, qw3, cus_per_xcd());
    a.n3 = plan.n3;
    a.n2 = plan.n2;
    const int64_t wgs = (int64_t)(a.n3 + a.n2) * pairs;
    const int64_t finish_waves = obs ? (int64_t)batch * n_groups * ((a.obs * n_rep + 15) / 16) : 0;
    if (wgs > INT32_MAX || (finish_waves + 3) / 4 > INT32_MAX) return UKV_ERR_INVALID_ARGUMENT;
    if (wgs > 0) {
      // With statistics, the prefill kernel writes the observation rows' (m, l) pairs and
      // obs_rows_finish_kernel, next on the same stream, turns them into the rows.
      if (dtype == UKV_DTYPE_BF16)
        hipLaunchKernelGGL((paged_prefill_kernel<UKV_DTYPE_BF16, W>), dim3((unsigned)wgs), dim3(64 * W), 0, stream, a);
      else
        hipLaunchKernelGGL((paged_prefill_kernel<UKV_DTYPE_F16, W>), dim3((unsigned)wgs), dim3(64 * W), 0, stream, a);
    }
    if (finish_waves > 0) {
      const dim3 fgrid((unsigned)((finish_waves + 3) / 4));
      if (dtype == UKV_DTYPE_BF16)
        hipLaunchKernelGGL(obs_rows_finish_kernel<UKV_DTYPE_BF16>, fgrid, dim3(256), 0, stream, a);
      else
        hipLaunchKernelGGL(obs_rows_finish_kernel<UKV_DTYPE_F16>, fgrid, dim3(256), 0, stream, a);
    }
  } else {
    const dim3 grid(total_q, num_q_heads);
    if (dtype == UKV_DTYPE_BF16)
      hipLaunchKernelGGL(paged_prefill_scalar_kernel<UKV_DTYPE_BF16>, grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(paged_prefill_scalar_kernel<UKV_DTYPE_F16>, grid, dim3(256), 0, stream, a);
    // The statistics come from the tiled kernel only: here every row is flagged, and the
    // scoring pass recomputes them from the keys.
    if (obs) {
      const int64_t rows = (int64_t)batch * num_q_heads * a.obs;
      if (rows > 0)
        hipLaunchKernelGGL(obs_flag_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, a, rows);
    }
  }
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}

}  // namespace

extern "C" int ukv_paged_prefill(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                                 const int32_t* cu_seqlens_q, const int32_t* kv_lens, void* out, int batch,
                                 int total_q, int max_chunk, int num_q_heads, int num_kv_heads, int head_dim,
                                 int n_rep, int max_blocks, int num_pages, const int64_t* q_strides,
                                 const int64_t* k_strides, const int64_t* v_strides, float softmax_scale,
                                 int dtype, ukv_stream_t stream_handle) {
  return prefill_impl(q, k_cache, v_cache, block_table, cu_seqlens_q, kv_lens, out, batch, total_q, max_chunk,
                      num_q_heads, num_kv_heads, head_dim, n_rep, max_blocks, num_pages, q_strides, k_strides,
                      v_strides, softmax_scale, dtype, stream_handle, nullptr);
}

extern "C" int ukv_paged_prefill_obs_stats(const void* q, const void* k_cache, const void* v_cache,
                                           const int32_t* block_table, const int32_t* cu_seqlens_q,
                                           const int32_t* kv_lens, void* out, int batch, int total_q, int max_chunk,
                                           int num_q_heads, int num_kv_heads, int head_dim, int n_rep,
                                           int max_blocks, int num_pages, const int64_t* q_strides,
                                           const int64_t* k_strides, const int64_t* v_strides,
                                           float softmax_scale, int dtype, int sink_len, int obs_len,
                                           float* obs_stats, int64_t stats_seq_stride, ukv_stream_t stream_handle) {
  if (sink_len < 0 || obs_len <= 0 || !obs_stats || (reinterpret_cast<uintptr_t>(obs_stats) & 7u) ||
      stats_seq_stride < (int64_t)num_q_heads * obs_len)
    return UKV_ERR_INVALID_ARGUMENT;
  const ObsStats st{obs_stats, stats_seq_stride, sink_len, obs_len};
  return prefill_impl(q, k_cache, v_cache, block_table, cu_seqlens_q, kv_lens, out, batch, total_q, max_chunk,
                      num_q_heads, num_kv_heads, head_dim, n_rep, max_blocks, num_pages, q_strides, k_strides,
                      v_strides, softmax_scale, dtype, stream_handle, &st);
}
