// Page16 paged decode attention for gfx950 (MI355X).
//
// Semantics follow core/page16_native.py:17-80 (BP-KV): for every sequence b and
// q head h, attend over tokens t < seqlens[b] whose K/V rows live at
// cache[block_table[b, t/16], t%16, h/n_rep, :], fp32 online softmax, output
// acc/l rounded to the input dtype.
//
// Work decomposition (split-K / flash-decoding):
//   * grid (G workgroups, 1, kv-group blocks), G = one per CU. The batch's
//     pages, sequence after sequence, form one list of P pages; share w
//     streams pages [w*P/G, (w+1)*P/G) - equal work for every workgroup however
//     ragged the lengths - crossing sequence boundaries as needed and leaving
//     one (m, l, acc) partial per sequence segment; each XCD runs a contiguous
//     run of shares. One wave per KV head (up to
//     eight per workgroup), so a workgroup reads each 32 KiB K page and V page
//     whole, and every KV byte is read exactly once for all n_rep q heads that
//     share it (GQA packing).
//   * both contractions run on the matrix cores: QK^T with
//     v_mfma_f32_16x16x32 (K rows as A, q heads as B columns) and P.V with
//     v_mfma_f32_16x16x16 (the QK result layout is the P operand layout, so P
//     never leaves the registers). P is split into two 16-bit parts so P.V keeps
//     fp32-grade weights.
//   * K and V rows go straight from HBM into registers with 16-byte loads; the
//     page of step p+1 is in flight while step p is reduced.
//   * online softmax in log2 units; the running max only moves when a score
//     exceeds it by more than 2^8, decided by a wave-wide vote.
//   * a second kernel merges each sequence's (m, l, acc) partials (log-sum-exp).
//
// A reference-faithful scalar kernel (natural exp, one workgroup per (b, h))
// serves shapes the split kernel is not instantiated for (head_dim not in
// {64, 128, 256}, n_rep > 16, or rows not 16-byte aligned).
#include <algorithm>
#include <atomic>
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
  float* part_o;     // [slots][Hq][D], slots = grid_wgs + B
  float2* part_ml;   // [slots][Hq]: (running max in log2 units, sum of exp2)
  int32_t* seq_start;  // [B] first global page of each sequence (written by workgroup 0)
  int32_t* seq_pages;  // [B] pages of each sequence
  int64_t q_sb, q_sh;
  int64_t k_sp, k_st, k_sh;
  int64_t v_sp, v_st, v_sh;
  int B, Hq, n_rep, n_groups, D, max_blocks, num_pages;
  int grid_wgs;      // G: workgroups sharing the batch's pages
  // Decode-token append (fused variant): k_new/v_new [B][n_groups][D] rows with
  // strides n_sb, n_sh; the token of sequence b goes to position lens[b] - 1.
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t n_sb, n_sh;
  float scale;       // natural-log units (scalar kernel)
  float scale_log2;  // scale * log2(e) (split kernel)
};

__device__ __forceinline__ int clamp_len(int L, int max_blocks) {
  const int cap = max_blocks * 16;
  return L < 0 ? 0 : (L > cap ? cap : L);
}

__device__ __forceinline__ int pages_of(int len, int max_blocks) { return (clamp_len(len, max_blocks) + 15) >> 4; }

__device__ __forceinline__ int wave_sum_i32(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ int wave_inclusive_scan_i32(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Splits fp32 softmax weights into two 16-bit parts (p ~= hi + lo, relative
// error below 2^-16) so that P.V can run on 16-bit MFMA with fp32-grade
// weights. The fp16 path scales p by 2^7 first so small weights stay normal.
template <int DT> struct PSplit;

template <> struct PSplit<UKV_DTYPE_BF16> {
  static constexpr float kScale = 1.f;
  static __device__ __forceinline__ uint32_t pack(float x0, float x1) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, bf16x2));
  }
  static __device__ __forceinline__ void split(const float (&p)[4], u32x2& hi, u32x2& lo) {
    hi = u32x2{pack(p[0], p[1]), pack(p[2], p[3])};
    const float r0 = p[0] - __uint_as_float(hi[0] << 16), r1 = p[1] - __uint_as_float(hi[0] & 0xffff0000u);
    const float r2 = p[2] - __uint_as_float(hi[1] << 16), r3 = p[3] - __uint_as_float(hi[1] & 0xffff0000u);
    lo = u32x2{pack(r0, r1), pack(r2, r3)};
  }
};

template <> struct PSplit<UKV_DTYPE_F16> {
  static constexpr float kScale = 128.f;
  static __device__ __forceinline__ uint32_t pack(float x0, float x1) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
  }
  static __device__ __forceinline__ void split(const float (&pin)[4], u32x2& hi, u32x2& lo) {
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = pin[r] * kScale;
    hi = u32x2{pack(p[0], p[1]), pack(p[2], p[3])};
    const float r0 = p[0] - Elem<UKV_DTYPE_F16>::lo(hi[0]), r1 = p[1] - Elem<UKV_DTYPE_F16>::hi(hi[0]);
    const float r2 = p[2] - Elem<UKV_DTYPE_F16>::lo(hi[1]), r3 = p[3] - Elem<UKV_DTYPE_F16>::hi(hi[1]);
    lo = u32x2{pack(r0, r1), pack(r2, r3)};
  }
};

#ifndef UKV_PAGE16_PIPE
#define UKV_PAGE16_PIPE 2
#endif
#ifndef UKV_PAGE16_NT
#define UKV_PAGE16_NT 1
#endif
#ifndef UKV_PAGE16_WAVES
#define UKV_PAGE16_WAVES 8
#endif
#ifndef UKV_PAGE16_MIN_WAVES_PER_EU
#define UKV_PAGE16_MIN_WAVES_PER_EU 1
#endif

// K/V page rows are read exactly once per call: optionally hint the loads as
// non-temporal so they do not displace cached lines.
__device__ __forceinline__ u32x4 ld16_stream(const uint16_t* p) {
  if constexpr (UKV_PAGE16_NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x2 ld8_stream(const uint16_t* p) {
  if constexpr (UKV_PAGE16_NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
  return *reinterpret_cast<const u32x2*>(p);
}

// V row fragment of one lane: DPL = D/16 consecutive dims of one token.
template <int DPL> struct VRow { uint32_t w[DPL / 2]; };

template <int DPL>
__device__ __forceinline__ void store_vrow(uint16_t* p, const VRow<DPL>& r) {
  if constexpr (DPL == 4) {
    *reinterpret_cast<u32x2*>(p) = u32x2{r.w[0], r.w[1]};
  } else {
#pragma unroll
    for (int c = 0; c < DPL / 8; ++c)
      *reinterpret_cast<u32x4*>(p + 8 * c) = u32x4{r.w[4 * c], r.w[4 * c + 1], r.w[4 * c + 2], r.w[4 * c + 3]};
  }
}

template <int DPL>
__device__ __forceinline__ void load_vrow(const uint16_t* p, VRow<DPL>& r) {
  if constexpr (DPL == 4) {
    const u32x2 x = ld8_stream(p);
    r.w[0] = x[0];
    r.w[1] = x[1];
  } else {
#pragma unroll
    for (int c = 0; c < DPL / 8; ++c) {
      const u32x4 x = ld16_stream(p + 8 * c);
      r.w[4 * c + 0] = x[0];
      r.w[4 * c + 1] = x[1];
      r.w[4 * c + 2] = x[2];
      r.w[4 * c + 3] = x[3];
    }
  }
}

// Split-K Page16 decode, one wave per KV head, all of that head's q heads
// (up to 16) per KV read.
//
// Lane l = (i16 = l % 16, kg = l / 16).
//   QK^T  v_mfma_f32_16x16x32: A = the page's K rows (row i16 = token, k-slots
//         dims 32*s + 8*kg .. +7), B = q^T (column i16 = q head, same dims).
//         Result: lane l holds S[token 4*kg + r][head i16], r = 0..3.
//         K is loaded like V (lane: tokens 4*kg .. +3, dims DPL*i16 ..), so that
//         each load instruction covers 4 whole token rows (4 x 256 B at D=128)
//         instead of 16 rows x 64 B, and goes through a wave-private LDS buffer
//         (4 row writes, then STEPS reads in the A layout) before the MFMAs;
//         measured 2 % faster at config 2 than loading the A layout directly.
//   P.V   v_mfma_f32_16x16x16: A = P (row i16 = head, k = tokens 4*kg .. +3),
//         which is exactly the QK result layout; B = V (k = tokens 4*kg .. +3,
//         column i16 -> dim DPL*i16 + e): each lane loads tokens 4*kg .. +3,
//         dims DPL*i16 .. +DPL-1 and v_perm_b32 regroups the 16-bit elements.
//         Result tile e: lane l holds O[head 4*kg + r][dim DPL*i16 + e].
// The running max is only moved when a score exceeds it by more than 2^8
// (log2 units; weights stay <= 256), decided by a wave-wide vote.
//
// APPEND: the decode token of sequence b (position lens[b] - 1) is taken from
// k_new/v_new instead of the pool. The wave that owns the page holding it loads
// the new K/V rows into registers of their own when its segment starts, swaps
// them in for the page's stale slot when that page is reduced, and stores them
// into the pool after its page loop (no memory operation is added inside the
// pipelined loop). Every (page, KV head) is read by exactly one wave, so each
// token row is written once, and the attention sees the same values as an
// append followed by a plain decode.
template <int DT, int D, bool APPEND>
__global__ void __launch_bounds__(64 * UKV_PAGE16_WAVES, UKV_PAGE16_MIN_WAVES_PER_EU) page16_split_kernel(const DecodeArgs a) {
  constexpr int STEPS = D / 32;  // QK k-steps of 32 dims
  constexpr int DPL = D / 16;    // V dims per lane = P.V output tiles
  constexpr float kTau = 8.f;
  constexpr int kPipe = D > 128 ? 1 : UKV_PAGE16_PIPE;  // D=256 has no registers for a second page

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int g = blockIdx.z * (blockDim.x >> 6) + wv;
  if (g >= a.n_groups) return;  // whole wave leaves; no workgroup barrier below
  const int G = a.grid_wgs;
  // Share w of the page list runs on workgroup blockIdx.x = 8 * (w % (G/8)) + w / (G/8): dispatch
  // puts workgroup i on XCD i % 8, so XCD x runs the contiguous shares x*G/8 .. (x+1)*G/8 - 1 and
  // the shares that carry one page more than the average (their positions follow P/G) spread evenly
  // over the XCDs instead of gathering on a few of them. Which workgroup runs a share does not
  // change its pages, slot or result.
  const int w = (G & 7) == 0 ? (int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const bool writer = blockIdx.x == 0 && blockIdx.z == 0 && wv == 0;

  // The batch's pages in sequence order form one list of P pages; workgroup w
  // takes pages [w*P/G, (w+1)*P/G), crossing sequence boundaries as needed.
  int P = 0;
  for (int c0 = 0; c0 < a.B; c0 += 64) {
    const int bb = c0 + lane;
    P += wave_sum_i32(bb < a.B ? pages_of(a.lens[bb], a.max_blocks) : 0);
  }
  const int x0 = (int)(((int64_t)w * P) / G);
  const int x1 = (int)(((int64_t)(w + 1) * P) / G);
  if (x0 >= x1 && !writer) return;

  // Exclusive prefix sums of pages per sequence; the sequence holding page x0.
  int b_first = -1, s_first = 0, carry = 0;
  for (int c0 = 0; c0 < a.B; c0 += 64) {
    const int bb = c0 + lane;
    const int n = bb < a.B ? pages_of(a.lens[bb], a.max_blocks) : 0;
    const int incl = wave_inclusive_scan_i32(n);
    const int start = carry + incl - n;
    if (writer && bb < a.B) {
      a.seq_start[bb] = start;
      a.seq_pages[bb] = n;
    }
    if (b_first < 0) {
      const uint64_t hit = __ballot(n > 0 && start + n > x0);
      if (hit) {
        const int l = __builtin_ctzll(hit);
        b_first = c0 + l;
        s_first = __builtin_amdgcn_readlane(start, l);
        if (!writer) break;
      }
    }
    carry += __builtin_amdgcn_readlane(incl, 63);
  }
  if (x0 >= x1) return;

  const int i16 = lane & 15;
  const int kg = lane >> 4;
  const int qh0 = g * a.n_rep;
  const int n_here = min(a.n_rep, a.Hq - qh0);
  const bool live = i16 < n_here;

  const uint16_t* kbase = a.k + (int64_t)(4 * kg) * a.k_st + (int64_t)g * a.k_sh + DPL * i16;
  // Wave-private LDS rows of the page's K (token-major): rows are loaded 4 tokens
  // x full width per instruction and read back in MFMA layout. The pitch of D + 16
  // elements (288 B at D = 128) keeps SQ_LDS_BANK_CONFLICT at 0 for the 16-row
  // reads (D + 8 conflicted on a quarter of the LDS cycles, at the same speed).
  constexpr int KP = D + 16;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[UKV_PAGE16_WAVES][16 * KP];
  uint16_t* ks = k_lds[wv];
  const uint16_t* vbase = a.v + (int64_t)(4 * kg) * a.v_st + (int64_t)g * a.v_sh + DPL * i16;

  // Per-segment state (one sequence's share of this workgroup's pages).
  int b = b_first;   // current sequence
  int L = 0;         // its attended tokens
  int pa = 0;        // first page of the segment (within the sequence)
  int pb = 0;        // one past the last page
  const int32_t* btrow = nullptr;
  int bid_win = 0;   // page ids pa + 64*k + lane of the current 64-page window
  int tail_page = -1;  // APPEND: page of the decode token if this segment holds it, else -1
  int tail_slot = 0;   // APPEND: its slot in that page
  int tail_pid = -1;   // APPEND: that page's id, -1 if invalid
  VRow<DPL> ktok;     // APPEND: the new K row (lanes kg == tail_slot / 4)
  VRow<DPL> vtok;      // APPEND: the new V row (lanes kg == tail_slot / 4)

  u32x4 qb[STEPS];   // B operand of QK^T: column i16 = q head qh0 + i16 (zero beyond n_here)
  float m_ref;       // running max of head i16 (log2 units)
  float lsum;        // this lane's share of that head's sum of weights
  f32x4 acc[DPL];

  auto load_page = [&](int p, VRow<DPL> (&kr)[4], VRow<DPL> (&vr)[4], int& nv) {
    const int idx = p - pa;
    if (idx != 0 && (idx & 63) == 0) bid_win = (p + lane < pb) ? btrow[p + lane] : 0;
    int bid = __builtin_amdgcn_readlane(bid_win, idx & 63);
    const bool ok = (unsigned)bid < (unsigned)a.num_pages;
    if constexpr (APPEND)
      if (p == tail_page) tail_pid = ok ? bid : -1;
    bid = ok ? bid : 0;
    nv = ok ? min(16, L - 16 * p) : 0;
    const uint16_t* kp = kbase + (int64_t)bid * a.k_sp;
#pragma unroll
    for (int t = 0; t < 4; ++t) load_vrow<DPL>(kp + (int64_t)t * a.k_st, kr[t]);
    const uint16_t* vp = vbase + (int64_t)bid * a.v_sp;
#pragma unroll
    for (int t = 0; t < 4; ++t) load_vrow<DPL>(vp + (int64_t)t * a.v_st, vr[t]);
  };

  // APPEND: on the token's page, its slot gets the new rows (per-lane register selects).
  auto swap_in_token = [&](VRow<DPL> (&kr)[4], VRow<DPL> (&vr)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bool mine = 4 * kg + t == tail_slot;
#pragma unroll
      for (int c = 0; c < DPL / 2; ++c) {
        kr[t].w[c] = mine ? ktok.w[c] : kr[t].w[c];
        vr[t].w[c] = mine ? vtok.w[c] : vr[t].w[c];
      }
    }
  };

  auto process_page = [&](const VRow<DPL> (&kr)[4], VRow<DPL> (&vr)[4], int nv) {
#pragma unroll
    for (int t = 0; t < 4; ++t) store_vrow<DPL>(ks + (4 * kg + t) * KP + DPL * i16, kr[t]);
    u32x4 ka[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) ka[s] = *reinterpret_cast<const u32x4*>(ks + i16 * KP + 8 * kg + 32 * s);
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) sacc = mfma16x16x32<DT>(ka[s], qb[s], sacc);
    float s2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) s2[r] = sacc[r] * a.scale_log2;
    if (nv < 16) {  // last page of the sequence or an invalid page id
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (4 * kg + r >= nv) {
          s2[r] = -INFINITY;
#pragma unroll
          for (int c = 0; c < DPL / 2; ++c) vr[r].w[c] = 0u;  // junk rows may be non-finite
        }
      }
    }
    const float mloc = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
    if (__any(mloc > m_ref + kTau)) {
      float mcol = fmaxf(mloc, __shfl_xor(mloc, 16));
      mcol = fmaxf(mcol, __shfl_xor(mcol, 32));
      const float m_new = fmaxf(m_ref, mcol);
      const float alpha = fast_exp2(m_ref - m_new);
      lsum *= alpha;
      m_ref = m_new;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * kg + r);
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e][r] *= ar;
      }
    }
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = fast_exp2(s2[r] - m_ref);
      lsum += p[r];
    }
    u32x2 phi, plo;
    PSplit<DT>::split(p, phi, plo);
#pragma unroll
    for (int c = 0; c < DPL / 2; ++c) {
      const u32x2 blo = {__builtin_amdgcn_perm(vr[1].w[c], vr[0].w[c], 0x05040100u),
                         __builtin_amdgcn_perm(vr[3].w[c], vr[2].w[c], 0x05040100u)};
      const u32x2 bhi = {__builtin_amdgcn_perm(vr[1].w[c], vr[0].w[c], 0x07060302u),
                         __builtin_amdgcn_perm(vr[3].w[c], vr[2].w[c], 0x07060302u)};
      acc[2 * c] = mfma16x16x16<DT>(phi, blo, acc[2 * c]);
      acc[2 * c] = mfma16x16x16<DT>(plo, blo, acc[2 * c]);
      acc[2 * c + 1] = mfma16x16x16<DT>(phi, bhi, acc[2 * c + 1]);
      acc[2 * c + 1] = mfma16x16x16<DT>(plo, bhi, acc[2 * c + 1]);
    }
  };

  constexpr float kUnscale = 1.f / PSplit<DT>::kScale;
  VRow<DPL> kb[kPipe][4];
  VRow<DPL> vb[kPipe][4];
  int nvb[kPipe];
  int seg_start = s_first;  // global index of page 0 of sequence b
  int x = x0;
  while (true) {
    const int n_b = pages_of(a.lens[b], a.max_blocks);
    L = clamp_len(a.lens[b], a.max_blocks);
    pa = x - seg_start;
    pb = min(x1, seg_start + n_b) - seg_start;
    btrow = a.bt + (int64_t)b * a.max_blocks;
    bid_win = (pa + lane < pb) ? btrow[pa + lane] : 0;
    if constexpr (APPEND) {
      // A length beyond the table is clamped; its token has no slot and is not written.
      tail_page = (L > 0 && L == a.lens[b]) ? ((L - 1) >> 4) : -1;
      if (tail_page < pa || tail_page >= pb) tail_page = -1;  // another workgroup's page
      tail_pid = -1;
      if (tail_page >= 0) {
        tail_slot = (L - 1) & 15;
        const uint16_t* kn = a.k_new + (int64_t)b * a.n_sb + (int64_t)g * a.n_sh;
        const uint16_t* vn = a.v_new + (int64_t)b * a.n_sb + (int64_t)g * a.n_sh;
        load_vrow<DPL>(kn + DPL * i16, ktok);
        load_vrow<DPL>(vn + DPL * i16, vtok);
      }
    }
    {
      const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(qh0 + (live ? i16 : 0)) * a.q_sh + 8 * kg;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) qb[s] = live ? ld16(qp + 32 * s) : u32x4{0u, 0u, 0u, 0u};
    }
    m_ref = kNegFltMax;
    lsum = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Software pipeline over PIPE register sets: while page p is reduced, the
    // loads of pages p+1 .. p+PIPE-1 are in flight.
#pragma unroll
    for (int i = 0; i < kPipe - 1; ++i)
      if (pa + i < pb) load_page(pa + i, kb[i], vb[i], nvb[i]);
    for (int base = pa; base < pb; base += kPipe) {
#pragma unroll
      for (int u = 0; u < kPipe; ++u) {
        const int p = base + u;
        if (p < pb) {
          const int nxt = (u + kPipe - 1) % kPipe;  // constant after unrolling
          if (p + kPipe - 1 < pb) load_page(p + kPipe - 1, kb[nxt], vb[nxt], nvb[nxt]);
          if constexpr (APPEND)
            if (p == tail_page) swap_in_token(kb[u], vb[u]);
          process_page(kb[u], vb[u], nvb[u]);
        }
      }
    }

    if constexpr (APPEND) {
      if (tail_pid >= 0) {  // the token's page is valid: write its rows into the pool
        if (kg == (tail_slot >> 2)) {
          store_vrow<DPL>(const_cast<uint16_t*>(kbase) + (int64_t)tail_pid * a.k_sp + (int64_t)(tail_slot & 3) * a.k_st,
                          ktok);
          store_vrow<DPL>(const_cast<uint16_t*>(vbase) + (int64_t)tail_pid * a.v_sp + (int64_t)(tail_slot & 3) * a.v_st,
                          vtok);
        }
      }
    }

    // Column sums of the weights: head i16 over the four token groups.
    float lcol = lsum + __shfl_xor(lsum, 16);
    lcol += __shfl_xor(lcol, 32);
    // Partial slot w + b is unique: a workgroup's sequences are consecutive and
    // a sequence's workgroups are consecutive.
    const int64_t slot = (int64_t)(w + b) * a.Hq + qh0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * kg + r;
      if (h < n_here) {
        f32x4* dst = reinterpret_cast<f32x4*>(a.part_o + (slot + h) * D + DPL * i16);
#pragma unroll
        for (int c = 0; c < DPL / 4; ++c)
          dst[c] = f32x4{acc[4 * c][r], acc[4 * c + 1][r], acc[4 * c + 2][r], acc[4 * c + 3][r]} * kUnscale;
      }
    }
    if (kg == 0 && live) a.part_ml[slot + i16] = make_float2(m_ref, lcol);

    x = seg_start + pb;
    if (x >= x1) break;
    seg_start += n_b;
    ++b;
    while (b < a.B && pages_of(a.lens[b], a.max_blocks) == 0) ++b;  // empty sequences hold no page
    if (b >= a.B) break;  // unreachable while x1 <= P; keeps every read inside the batch
  }
}

__device__ __forceinline__ float block_reduce_256(float x, float* red, bool is_max) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float y = __shfl_xor(x, o);
    x = is_max ? fmaxf(x, y) : x + y;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  __syncthreads();
  return r;
}

// Merges the partials of one (sequence, q head): log-sum-exp in log2 units.
// The sequence's pages [S, S+n) of the batch's P pages were split over
// workgroups w = floor(((S+1)G - 1)/P) .. floor(((S+n)G - 1)/P), whose partials
// sit in slots w + b. 256 threads: thread (cs, dq) owns float4 dims 4*dq.. of
// partials cs, cs+CS, ...; it issues the loads of its first kPre rows together
// with the (m, l) loads, so that one memory round trip serves both; the weights
// are computed once into LDS, and the CS partial sums meet in LDS.
template <int DT, int D>
__global__ void __launch_bounds__(256) page16_combine_kernel(const DecodeArgs a) {
  constexpr int TD = D / 4;       // threads per partial row (float4 each)
  constexpr int CS = 256 / TD;    // chunk groups
  constexpr int kPre = 4;         // partial rows per thread loaded before the weights
  extern __shared__ float w_s[];  // [grid_wgs] weights, then [CS][D] sums
  __shared__ float red[4];

  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int n_pages = a.seq_pages[b];
  const int64_t P = (int64_t)a.seq_start[a.B - 1] + a.seq_pages[a.B - 1];
  const int64_t S = a.seq_start[b];
  const int G = a.grid_wgs;
  const int w_first = n_pages > 0 ? (int)(((S + 1) * G - 1) / P) : 0;
  const int w_last = n_pages > 0 ? (int)(((S + n_pages) * G - 1) / P) : -1;
  const int n_chunks = w_last - w_first + 1;
  const int64_t base = (int64_t)(w_first + b) * a.Hq + h;
  // With fewer pages than workgroups (P < G) some workgroups in [w_first, w_last]
  // own no page and wrote no partial: their slots hold stale data and are skipped.
  auto owns_pages = [&](int c) {
    const int64_t w = w_first + c;
    return ((w + 1) * P) / G > (w * P) / G;
  };

  const int cs = tid / TD;
  const int dq = tid % TD;
  const float* po = a.part_o + base * D + 4 * dq;
  const int64_t cstride = (int64_t)a.Hq * D;
  f32x4 rows[kPre];  // partials cs + k*CS (in the workspace even when stale; skipped below)
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
    const int c = cs + k * CS;
    rows[k] = c < n_chunks ? *reinterpret_cast<const f32x4*>(po + (int64_t)c * cstride) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bool own0 = tid < n_chunks && owns_pages(tid);
  const float2 ml0 = own0 ? a.part_ml[base + (int64_t)tid * a.Hq] : make_float2(-INFINITY, 0.f);

  float mx = ml0.x;
  for (int c = tid + 256; c < n_chunks; c += 256)
    if (owns_pages(c)) mx = fmaxf(mx, a.part_ml[base + (int64_t)c * a.Hq].x);
  const float M = block_reduce_256(mx, red, true);
  float dsum = 0.f;
  for (int c = tid; c < n_chunks; c += 256) {
    const bool own = c == tid ? own0 : owns_pages(c);
    if (!own) {
      w_s[c] = -1.f;  // marks an empty slot (real weights are >= 0 or NaN)
      continue;
    }
    const float2 ml = c == tid ? ml0 : a.part_ml[base + (int64_t)c * a.Hq];
    const float w = exp2f(ml.x - M);
    w_s[c] = w;
    dsum += ml.y * w;
  }
  const float den = block_reduce_256(dsum, red, false);  // also orders the w_s writes

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
    const int c = cs + k * CS;
    if (c < n_chunks) {
      const float w = w_s[c];
      if (!(w < 0.f)) acc += w * rows[k];
    }
  }
#pragma unroll 4
  for (int c = cs + kPre * CS; c < n_chunks; c += CS) {
    const float w = w_s[c];
    if (!(w < 0.f)) acc += w * *reinterpret_cast<const f32x4*>(po + (int64_t)c * cstride);
  }
  float* sums = w_s + ((a.grid_wgs + 3) & ~3);
  *reinterpret_cast<f32x4*>(sums + cs * D + 4 * dq) = acc;
  __syncthreads();
  if (tid < D) {
    float num = 0.f;
#pragma unroll
    for (int g = 0; g < CS; ++g) num += sums[g * D + tid];
    a.out[((int64_t)b * a.Hq + h) * D + tid] = Elem<DT>::from_float(n_chunks > 0 ? num / den : NAN);
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

constexpr int kMinPagesPerWg = 8;  // below this a workgroup's setup outweighs its pages

// CU count of the current device, cached per device id (0 = not yet read; a
// racing first read stores the same value twice).
int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// UKV_PAGE16_WGS, read once per process (0 when unset or not a positive number).
int env_wgs() {
  static const int v = [] {
    const char* env = std::getenv("UKV_PAGE16_WGS");
    const int x = (env && *env) ? std::atoi(env) : 0;
    return x > 0 ? std::min(x, 65535) : 0;
  }();
  return v;
}

// Workgroups G sharing the batch's pages: one per CU (a single round of equal
// workgroups measured fastest), fewer when even the largest possible batch
// (batch * max_blocks pages) gives each fewer than kMinPagesPerWg pages;
// UKV_PAGE16_WGS overrides it for launch-shape sweeps.
int split_wgs_for(int batch, int max_blocks) {
  if (const int v = env_wgs()) return v;
  const long long bound = (long long)batch * (long long)std::max(max_blocks, 1);
  const long long g = std::min<long long>(device_cu_count(), (bound + kMinPagesPerWg - 1) / kMinPagesPerWg);
  return (int)std::max<long long>(1, g);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct WorkspaceLayout {
  size_t part_o_off, part_ml_off, seq_off, total;
  int wgs;
};

// [slots][Hq][D] fp32 partials, [slots][Hq] (m, l), then the per-sequence page
// starts and counts; slots = G + batch.
WorkspaceLayout workspace_layout(int batch, int hq, int d, int max_blocks) {
  WorkspaceLayout w{};
  w.wgs = split_wgs_for(batch, max_blocks);
  const size_t slots = ((size_t)w.wgs + (size_t)batch) * hq;
  w.part_o_off = 0;
  w.part_ml_off = align256(slots * d * sizeof(float));
  w.seq_off = w.part_ml_off + align256(slots * sizeof(float2));
  w.total = w.seq_off + align256(2 * (size_t)batch * sizeof(int32_t));
  return w;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT, int D>
void launch_split(const DecodeArgs& a, hipStream_t stream) {
  const int waves = std::min(UKV_PAGE16_WAVES, a.n_groups);
  const dim3 grid(a.grid_wgs, 1, (a.n_groups + waves - 1) / waves);
  if (a.k_new)
    hipLaunchKernelGGL((page16_split_kernel<DT, D, true>), grid, dim3(64 * waves), 0, stream, a);
  else
    hipLaunchKernelGGL((page16_split_kernel<DT, D, false>), grid, dim3(64 * waves), 0, stream, a);
}

template <int DT>
void launch_combine_dt(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid(a.Hq, a.B);
  const size_t lds = (size_t)(((a.grid_wgs + 3) & ~3) + 256 * 4) * sizeof(float);
  switch (a.D) {
    case 64: hipLaunchKernelGGL((page16_combine_kernel<DT, 64>), grid, dim3(256), lds, stream, a); break;
    case 128: hipLaunchKernelGGL((page16_combine_kernel<DT, 128>), grid, dim3(256), lds, stream, a); break;
    default: hipLaunchKernelGGL((page16_combine_kernel<DT, 256>), grid, dim3(256), lds, stream, a); break;
  }
}

void launch_combine(const DecodeArgs& a, int dtype, hipStream_t stream) {
  if (dtype == UKV_DTYPE_BF16)
    launch_combine_dt<UKV_DTYPE_BF16>(a, stream);
  else
    launch_combine_dt<UKV_DTYPE_F16>(a, stream);
}

template <int DT>
bool dispatch_split(const DecodeArgs& a, hipStream_t stream) {
  if (a.n_rep > 16) return false;
  switch (a.D) {
    case 64: launch_split<DT, 64>(a, stream); return true;
    case 128: launch_split<DT, 128>(a, stream); return true;
    case 256: launch_split<DT, 256>(a, stream); return true;
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

namespace {

// The decode token of the fused entry point: rows k_new[b], v_new[b] of
// [batch][num_kv_heads][head_dim] with element strides new_strides[0..1].
struct TokenRows {
  const void* k;
  const void* v;
  const int64_t* strides;
};

int decode_impl(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                const int32_t* seqlens, void* out, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                int n_rep, int max_blocks, int num_pages, const int64_t* q_strides, const int64_t* k_strides,
                const int64_t* v_strides, float softmax_scale, int dtype, void* workspace, size_t workspace_bytes,
                ukv_stream_t stream_handle, const TokenRows* tok) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0) return UKV_ERR_EMPTY;
  if (head_dim > 256) return UKV_ERR_HEAD_DIM;
  if (dtype != UKV_DTYPE_F16 && dtype != UKV_DTYPE_BF16) return UKV_ERR_DTYPE;
  if (num_kv_heads <= 0 || n_rep < 1) return UKV_ERR_GQA;
  const int n_groups = (num_q_heads + n_rep - 1) / n_rep;
  if (n_groups > num_kv_heads) return UKV_ERR_GQA;
  if (max_blocks < 0 || num_pages < 0) return UKV_ERR_INVALID_ARGUMENT;
  if (!q || !out || !seqlens || !q_strides || !k_strides || !v_strides) return UKV_ERR_INVALID_ARGUMENT;
  if (max_blocks > 0 && (!block_table || !k_cache || !v_cache || num_pages <= 0)) return UKV_ERR_INVALID_ARGUMENT;
  if (tok && (!tok->k || !tok->v || !tok->strides)) return UKV_ERR_INVALID_ARGUMENT;

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
  // The split kernel writes the token itself when every KV head is read by
  // some wave and the new rows are 16-byte aligned; otherwise the append runs
  // as its own kernel first.
  const bool fused = tok && fast && n_groups == num_kv_heads && aligned16(tok->k) && aligned16(tok->v) &&
                     tok->strides[0] % 8 == 0 && tok->strides[1] % 8 == 0;
  WorkspaceLayout w{};
  if (fast) {
    w = workspace_layout(batch, num_q_heads, head_dim, max_blocks);
    if (!workspace || workspace_bytes < w.total || !aligned16(workspace)) return UKV_ERR_WORKSPACE;
  }
  if (tok && !fused && max_blocks > 0) {
    const int rc = append_decode_rows(const_cast<void*>(k_cache), const_cast<void*>(v_cache), k_strides, v_strides,
                                      tok->k, tok->v, tok->strides, block_table, max_blocks, seqlens, -1, nullptr,
                                      batch, 16, num_kv_heads, head_dim, num_pages, stream);
    if (rc != UKV_OK) return rc;
  }

  if (fast) {
    char* ws = static_cast<char*>(workspace);
    a.part_o = reinterpret_cast<float*>(ws + w.part_o_off);
    a.part_ml = reinterpret_cast<float2*>(ws + w.part_ml_off);
    a.seq_start = reinterpret_cast<int32_t*>(ws + w.seq_off);
    a.seq_pages = a.seq_start + batch;
    a.grid_wgs = w.wgs;
    if (fused) {
      a.k_new = static_cast<const uint16_t*>(tok->k);
      a.v_new = static_cast<const uint16_t*>(tok->v);
      a.n_sb = tok->strides[0];
      a.n_sh = tok->strides[1];
    }
    const bool launched =
        dtype == UKV_DTYPE_BF16 ? dispatch_split<UKV_DTYPE_BF16>(a, stream) : dispatch_split<UKV_DTYPE_F16>(a, stream);
    if (!launched) return UKV_ERR_LAUNCH;
    if (hipGetLastError() != hipSuccess) return UKV_ERR_LAUNCH;
    launch_combine(a, dtype, stream);
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

}  // namespace

extern "C" int ukv_page16_decode(const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* block_table, const int32_t* seqlens, void* out, int batch,
                                 int num_q_heads, int num_kv_heads, int head_dim, int n_rep, int max_blocks,
                                 int num_pages, const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, float softmax_scale, int dtype, void* workspace,
                                 size_t workspace_bytes, ukv_stream_t stream_handle) {
  return decode_impl(q, k_cache, v_cache, block_table, seqlens, out, batch, num_q_heads, num_kv_heads, head_dim,
                     n_rep, max_blocks, num_pages, q_strides, k_strides, v_strides, softmax_scale, dtype, workspace,
                     workspace_bytes, stream_handle, nullptr);
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the split-K workspace lives in a file-scope device
// array instead of a caller buffer. Each GPU holds its own copy of the array
// (UKV_PAGE16_SCRATCH_BYTES, for the life of the process) at its own address;
// host code reaches it only through the address hipGetSymbolAddress reports for
// the current device, read once per device on the first call there. Calls that
// overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[UKV_PAGE16_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device (nullptr on failure).
void* scratch_address() {
  static std::atomic<void*> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  void* p = cached[dev].load(std::memory_order_acquire);
  if (p) return p;
  // Racing first calls on one device store the same address.
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
  cached[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace

extern "C" int ukv_page16_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                         const int32_t* block_table, const int32_t* seqlens, void* out, int batch,
                                         int num_q_heads, int num_kv_heads, int head_dim, int n_rep, int max_blocks,
                                         int num_pages, const int64_t* q_strides, const int64_t* k_strides,
                                         const int64_t* v_strides, float softmax_scale, int dtype,
                                         ukv_stream_t stream_handle) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0) return UKV_ERR_EMPTY;
  if (ukv_page16_workspace_bytes(batch, num_q_heads, head_dim, max_blocks) > UKV_PAGE16_SCRATCH_BYTES)
    return UKV_ERR_WORKSPACE;
  void* ws = scratch_address();
  if (!ws) return UKV_ERR_NO_DEVICE;
  return decode_impl(q, k_cache, v_cache, block_table, seqlens, out, batch, num_q_heads, num_kv_heads, head_dim,
                     n_rep, max_blocks, num_pages, q_strides, k_strides, v_strides, softmax_scale, dtype, ws,
                     UKV_PAGE16_SCRATCH_BYTES, stream_handle, nullptr);
}

extern "C" int ukv_page16_decode_append(const void* q, void* k_cache, void* v_cache, const int32_t* block_table,
                                        const int32_t* seqlens, const void* k_new, const void* v_new,
                                        const int64_t* new_strides, void* out, int batch, int num_q_heads,
                                        int num_kv_heads, int head_dim, int n_rep, int max_blocks, int num_pages,
                                        const int64_t* q_strides, const int64_t* k_strides,
                                        const int64_t* v_strides, float softmax_scale, int dtype, void* workspace,
                                        size_t workspace_bytes, ukv_stream_t stream_handle) {
  const TokenRows tok{k_new, v_new, new_strides};
  return decode_impl(q, k_cache, v_cache, block_table, seqlens, out, batch, num_q_heads, num_kv_heads, head_dim,
                     n_rep, max_blocks, num_pages, q_strides, k_strides, v_strides, softmax_scale, dtype, workspace,
                     workspace_bytes, stream_handle, &tok);
}
