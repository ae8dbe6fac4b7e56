// SnapKV observation-window block scores for gfx950 (MI355X).
//
// For every item (one layer of one sequence) this computes what
// core/scheduler.py:565-592 (_score_layer_blocks_for_selection) computes:
//   K_mid = K[:, sink : L - obs, :], zero-padded to a multiple of the block size
//   A     = softmax(Q_obs . repeat_kv(K_mid)^T * scale)      [H_q, obs, aligned]
//   s     = A.mean(over obs queries).max(over q heads)       [aligned]
//   block = s.view(N, block).sum(-1);  maxpool1d(k=3, s=1, p=1) when N >= 3
// from 16-bit Q and K (the reference runs these steps in the model dtype).
// Scores, maxima and sums are fp32; each softmax weight is rounded to fp16
// (relative error <= 2^-11, scaled by a power of two away from fp16's subnormal
// range) where the matrix cores sum it.
//
// Work decomposition: an item's mid keys form Kt tiles of 64 keys, split into
// S contiguous ranges; one workgroup (8 waves) per (range, item). A unit is
// one KV group's q heads, or part of them when n_rep * obs > 512 rows: the
// unit's Q rows (up to 512 = 8 waves x 4 tiles of 16) stay in registers while
// its K tiles stream through LDS (64 keys, 16-byte rows loaded once per
// workgroup, padded pitch against bank conflicts). The scores run on
// v_mfma_f32_16x16x32.
//   pass 1 (stats): per query row, running max and sum of exp2 over the
//           range's keys -> partial (m, l) per (range, row); a small kernel
//           merges the ranges into m' = m + log2(l);
//   pass 2 (scores): p = exp2(s - m'), summed over each head's queries (on
//           the matrix cores per wave, then the head's waves in a fixed order
//           through LDS, so results are reproducible), max over heads, running
//           max over units per key in LDS, then the sums over 16-key blocks of
//           the range;
//   finish: the 3-wide max pool over each item's blocks.
// Both passes compute Q K^T, so the cost is 2 * (2 * H_q * obs * aligned * D)
// FLOPs per item on the matrix cores; K is read twice.
//
// A scalar path (one thread per query row, plain loops) serves shapes the
// tiled kernel is not instantiated for (head_dim not 64/128, obs not a
// multiple of 16 or above 512, rows not 16-byte aligned).
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "ukv_common.h"

namespace ukv {


#ifndef UKV_SNAP_WAVES
#define UKV_SNAP_WAVES 8  // waves per workgroup
#endif
#ifndef UKV_SNAP_MAX_KEYS
#define UKV_SNAP_MAX_KEYS 8192  // keys per range (LDS running max)
#endif

constexpr int kSnapWaves = UKV_SNAP_WAVES;
constexpr int kSnapTile = 64;                     // keys per LDS tile
constexpr int kSnapMaxTW = 4;                     // row tiles of 16 per wave
constexpr int kSnapMaxKeys = UKV_SNAP_MAX_KEYS;

struct SnapArgs {
  const uint16_t* q;  // [items][H_q][obs][D] with strides q_si, q_sh, q_st
  int64_t q_si, q_sh, q_st;
  const uint16_t* k;  // token t, head g of item (b, l): see key_row() (pages hold 16 tokens)
  int64_t k_sl, k_sb, k_st, k_sh;
  const int32_t* table;  // [seqs][max_blocks] or null (dense)
  int max_blocks, num_pages;
  int layers, items;
  int sink, obs, L_mid, aligned, n_blocks;
  int Hq, Hkv, n_rep, D;
  int hp, parts;         // q heads per unit, units per KV group
  int S, Kt;             // key ranges per item, 64-key tiles per item
  float scale_log2;
  float2* part_stats;    // [items][S][Hq*obs] (m, l) per range
  float2* stats;         // [items][Hq*obs] (m + log2(l), unused)
  float* raw;            // [items][n_blocks] block sums before pooling
  int32_t* redo;         // [items] or null: pass 1 and the merge run only for items with redo != 0
  float* out;            // [items][out_stride]
  int64_t out_stride;
};

// Element offset of the K row of mid key j (token sink + j), head g, item
// (b = item / layers, l = item % layers); -1 for a zero row (padding or an
// invalid page id).
__device__ __forceinline__ int64_t key_row(const SnapArgs& a, int item, int j, int g) {
  if (j >= a.L_mid) return -1;
  const int b = item / a.layers, l = item % a.layers;
  const int t = a.sink + j;
  int64_t off = (int64_t)l * a.k_sl + (int64_t)g * a.k_sh;
  if (a.table) {
    const int blk = t >> 4;
    if (blk >= a.max_blocks) return -1;
    const int page = a.table[(int64_t)b * a.max_blocks + blk];
    if ((unsigned)page >= (unsigned)a.num_pages) return -1;
    off += (int64_t)page * a.k_sb + (int64_t)(t & 15) * a.k_st;
  } else {
    off += (int64_t)b * a.k_sb + (int64_t)t * a.k_st;
  }
  return off;
}

// Max of x over the lanes l, l^16, l^32, l^48 (the 4 lane groups of a wave),
// with the gfx950 cross-row swaps (no LDS traffic).
__device__ __forceinline__ float max_lane_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));  // x, x^16
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));  // and the other 32-lane half
}

template <int D> struct SnapLds {
  static constexpr int kPitch = D + 16;  // elements per key row in LDS
  alignas(16) uint16_t kt[2][kSnapTile * kPitch];  // double-buffered K tiles (ds_read_b128 / ds_write_b128)
  float colpart[2][32][kSnapTile];       // double-buffered column sums per wave, at its first row tile
  float colmax[kSnapMaxKeys];            // running max over units, per key of the range
};

// TW: row tiles of 16 per wave (1, 2 or 4); TW divides the tiles of one q head,
// so a wave's tiles belong to one head.
//
//   pass 1 (S^T: lane l holds keys 4*(l/16) + r of column tile ct for query
//          column l%16 of row tile k) keeps a running max per query column, the
//          same in the 4 lane groups. A step's weights are computed under the
//          current max; only when a wave-wide vote finds one above 2^8 (or an
//          overflow, as on the first tile) is the exact max taken and the column
//          rescaled. The weights are summed over keys on the matrix cores: as fp16
//          B operand against an all-ones A, every row of the result is the sum.
//   pass 2 (S: lane l holds query rows 4*(l/16) + r of key l%16) gets
//          m' = m + log2(l) per row, so p = exp2(s * scale - m') is one FMA and
//          one exp2; the weights are summed over the wave's rows on the matrix
//          cores (fp16 B operand against a one-hot selector A that puts column
//          tile ct's sums into row 4*ct); the waves of a head are added and the
//          max over heads taken by 64 * hp threads.
// K tiles and column sums are double-buffered: one barrier per tile.
template <int DT, int D, bool SCORES, int TW>
__global__ void __launch_bounds__(64 * kSnapWaves, 2) snap_tile_kernel(const SnapArgs a) {
  constexpr int STEPS = D / 32;
  constexpr int CHUNKS = kSnapTile * D / 8;  // 16-byte chunks per K tile
  constexpr int CPT = CHUNKS / (64 * kSnapWaves);
  // Weights enter the column-sum MFMAs as fp16 times a power of two: pass 1
  // keeps them at or below 2^8 (2^15 lifted), pass 2's are at most 1 (2^14
  // lifted); the lift keeps small weights out of fp16's subnormal range.
  constexpr float kLift1 = 7.f, kLift2 = 14.f, kUnlift2 = 1.f / 16384.f;
  static_assert(CHUNKS % (64 * kSnapWaves) == 0, "tile chunks must divide over the threads");
  __shared__ SnapLds<D> lds;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int s = blockIdx.x, item = blockIdx.y;
  if (!SCORES && a.redo && a.redo[item] == 0) return;  // whole workgroup: statistics given
  const int t0 = (int)((int64_t)s * a.Kt / a.S), t1 = (int)((int64_t)(s + 1) * a.Kt / a.S);
  const int key0 = t0 * kSnapTile;
  const int R = a.hp * a.obs;  // rows of a unit
  const int T = R / 16;        // row tiles of a unit
  const int tph = a.obs / 16;  // row tiles per q head
  const int rows_all = a.Hq * a.obs;
  const float c = a.scale_log2;
  const bool hp_pow2 = (a.hp & (a.hp - 1)) == 0;
  const int hp_log2 = 31 - __builtin_clz(a.hp);
  const int item_b = item / a.layers, item_l = item - item_b * a.layers;  // sequence, layer
  const int32_t* trow = a.table ? a.table + (int64_t)item_b * a.max_blocks : nullptr;
  // The kernel never writes the table: read it through the constant address space, so that
  // wave-uniform ids come through the scalar cache.
  typedef const __attribute__((address_space(4))) int32_t cint32;
  cint32* trow_c = (cint32*)trow;
  // MFMA A operands of the column sums (fp16 1.0 pairs): all ones (pass 1), and
  // rows 0 and 4 selecting dwords 0-1 and 2-3 of the B operand (pass 2).
  constexpr uint32_t kOnes = 0x3C003C00u;
  const u32x4 ones = u32x4{kOnes, kOnes, kOnes, kOnes};
  const u32x4 colsel = u32x4{l16 == 0 ? kOnes : 0u, l16 == 0 ? kOnes : 0u, l16 == 4 ? kOnes : 0u,
                             l16 == 4 ? kOnes : 0u};

  if constexpr (SCORES)
    for (int i = tid; i < (t1 - t0) * kSnapTile; i += blockDim.x) lds.colmax[i] = 0.f;

  for (int u = 0; u < a.Hkv * a.parts; ++u) {
    const int g = u / a.parts;
    const int h0 = g * a.n_rep + (u % a.parts) * a.hp;  // first q head of the unit

    // This wave's row tiles: w*TW .. w*TW+TW-1 (tiles past T are zero and unused).
    u32x4 qa[TW][STEPS];
    // pass 1: m[k][0] is kLift1 minus the running max (log2 units) of query column
    //         l16 of tile k, the same in the 4 lane groups, and every row of lsum[k]
    //         holds 2^kLift1 times the column's running sum of weights;
    // pass 2: m[k][r] = m' - kLift2 of query row 4*lg + r of tile k.
    float m[TW][4];
    f32x4 lsum[TW];
#pragma unroll
    for (int k = 0; k < TW; ++k) {
      lsum[k] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int tile = wv * TW + k;
      const bool on = tile < T;
      const int rr = tile * 16 + l16;  // A row of this lane
      const uint16_t* qp = a.q + (int64_t)item * a.q_si + (int64_t)(h0 + rr / a.obs) * a.q_sh +
                           (int64_t)(rr % a.obs) * a.q_st + 8 * lg;
#pragma unroll
      for (int st = 0; st < STEPS; ++st) qa[k][st] = on ? ld16(qp + 32 * st) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        m[k][r] = INFINITY;  // pass 1: kLift1 - max with max = -inf; pass 2: rows past the unit weigh 0
        if constexpr (SCORES) {
          if (on) {  // C rows 4*lg + r of the tile
            const int row = tile * 16 + 4 * lg + r;
            m[k][r] = a.stats[(int64_t)item * rows_all + (int64_t)(h0 + row / a.obs) * a.obs + row % a.obs].x -
                      kLift2;
          }
        }
      }
    }

    // K tile loads: thread chunk cc = tid + i*512 -> key cc / (D/8), dims 8*(cc % (D/8)).
    // key_row() with the item's and the unit's terms taken out of the tile loop.
    const uint16_t* kg = a.k + (int64_t)item_l * a.k_sl + (int64_t)g * a.k_sh;
    u32x4 pre[CPT];
    // Per chunk, the thread's key offset in a tile, its token's slot in a page and its
    // page relative to the wave's first page are the same for every tile (a tile is 64
    // keys = 4 pages), so only the wave-uniform page ids change from tile to tile.
    int64_t roff[CPT];  // element offset of the chunk within its page (paged) or tile (dense)
    bool second[CPT];   // paged: the chunk's key is on the wave's second page
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int cc = tid + i * 64 * kSnapWaves;
      const int kk = cc / (D / 8), kk0 = __builtin_amdgcn_readfirstlane(kk);
      const int t = a.sink + kk;  // token of the key in tile 0 (tile u adds 64u = 4u pages)
      second[i] = (t >> 4) != ((a.sink + kk0) >> 4);
      roff[i] = (trow ? (int64_t)(t & 15) * a.k_st : (int64_t)t * a.k_st) + 8 * (cc % (D / 8));
    }
    auto fetch = [&](int tile_idx) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int cc = tid + i * 64 * kSnapWaves;
        const int j = tile_idx * kSnapTile + cc / (D / 8);  // mid key
        const uint16_t* src = nullptr;
        if (trow) {
          // A wave's keys (64 / (D/8) <= 8 consecutive ones) lie in at most two pages:
          // their ids are read once per wave through the scalar cache.
          const int blk_a = (a.sink + __builtin_amdgcn_readfirstlane(j)) >> 4;
          const int id_a = blk_a < a.max_blocks ? trow_c[blk_a] : -1;
          const int id_b = blk_a + 1 < a.max_blocks ? trow_c[blk_a + 1] : -1;
          const int page = second[i] ? id_b : id_a;
          if (j < a.L_mid && (unsigned)page < (unsigned)a.num_pages)
            src = kg + (int64_t)page * a.k_sb + roff[i];
        } else if (j < a.L_mid) {
          src = kg + (int64_t)item_b * a.k_sb + (int64_t)tile_idx * kSnapTile * a.k_st + roff[i];
        }
        pre[i] = src ? ld16(src) : u32x4{0u, 0u, 0u, 0u};
      }
    };
    auto stash = [&](int buf) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int cc = tid + i * 64 * kSnapWaves;
        *reinterpret_cast<u32x4*>(&lds.kt[buf][(cc / (D / 8)) * SnapLds<D>::kPitch + 8 * (cc % (D / 8))]) = pre[i];
      }
    };

    // Per (key, head) of tile `tile`: add the head's waves' column sums (fixed order),
    // take the max over the unit's heads, and fold it into the range's running max.
    auto head_sum = [&](int tile, int b) {
      const int kb0 = tile * kSnapTile - key0;
      if (hp_pow2 && kSnapTile * a.hp <= (int)blockDim.x) {
        if (tid < kSnapTile * a.hp) {
          const int key = tid >> hp_log2, h = tid & (a.hp - 1);
          float x = 0.f;
          for (int q = h * tph; q < (h + 1) * tph; q += TW) x += lds.colpart[b][q][key];
          for (int o = 1; o < a.hp; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));  // hp consecutive lanes
          if (h == 0) lds.colmax[kb0 + key] = fmaxf(lds.colmax[kb0 + key], x);
        }
      } else if (tid < kSnapTile) {
        float mx = 0.f;
        for (int h = 0; h < a.hp; ++h) {
          float x = 0.f;
          for (int q = h * tph; q < (h + 1) * tph; q += TW) x += lds.colpart[b][q][tid];
          mx = fmaxf(mx, x);
        }
        lds.colmax[kb0 + tid] = fmaxf(lds.colmax[kb0 + tid], mx);
      }
    };

    __syncthreads();  // the previous unit is done with both buffers
    fetch(t0);
    stash(0);
    if (t0 + 1 < t1) fetch(t0 + 1);
    __syncthreads();
    for (int ti = t0; ti < t1; ++ti) {
      const int buf = (ti - t0) & 1;
      const int kbase = ti * kSnapTile;
      // Keys at or past the padded end lie in the last tile of an item only; a
      // 16-key column tile is either wholly valid or wholly past it (aligned % 16 == 0).
      // The tile runs in steps j = (half, row tile k): the 32 keys of column tiles
      // 2*half, 2*half + 1 against row tile k. K operands (key l16 of column tile
      // ct, dims 8*lg + 32*st) are read from LDS once per half. Pass 2 computes
      // S = Q K^T (lane: query rows 4*lg + r of key l16), pass 1 S^T = K Q^T (lane:
      // keys 4*lg + r of query l16); the 16x16x32 A and B operand layouts are the
      // same, so only the operand order differs. Step j+1's scores are issued on
      // the matrix cores before step j's weights are computed on the vector ALUs.
      // pass 2: rows 0 and 4 of colsum[half] hold the column sums of column tiles
      // 2*half and 2*half + 1 over the wave's row tiles (one q head), i.e.
      // element 0 of lanes 0-31 of colsum[half].
      f32x4 colsum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      {
        constexpr int NSTEP = 2 * TW;
        u32x4 kb[2][STEPS];
        auto load_half = [&](int hf) {
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
            for (int st = 0; st < STEPS; ++st)
              kb[c2][st] = *reinterpret_cast<const u32x4*>(
                  &lds.kt[buf][((2 * hf + c2) * 16 + l16) * SnapLds<D>::kPitch + 8 * lg + 32 * st]);
        };
        f32x4 acc[2][2];
        auto scores = [&](int j, f32x4(&dst)[2]) {
          const int k = j % TW;
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2) {
            dst[c2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < STEPS; ++st)
              dst[c2] = SCORES ? mfma16x16x32<DT>(qa[k][st], kb[c2][st], dst[c2])
                               : mfma16x16x32<DT>(kb[c2][st], qa[k][st], dst[c2]);
          }
        };
        load_half(0);
        scores(0, acc[0]);
#pragma unroll
        for (int j = 0; j < NSTEP; ++j) {
          const int hf = j / TW, k = j % TW;
          if (j + 1 < NSTEP) {
            if ((j + 1) % TW == 0) load_half((j + 1) / TW);
            scores(j + 1, acc[(j + 1) & 1]);
          }
          // The previous tile's head sums (its column sums were written before the last
          // barrier; that buffer is written again only after the next one), while the
          // scores above run on the matrix cores.
          if constexpr (SCORES)
            if (j == 0 && ti > t0) head_sum(ti - 1, buf ^ 1);
          f32x4(&sc)[2] = acc[j & 1];
          // The step's weights run at raised wave priority, lowered again for their column-sum
          // MFMA (two-pass call ~1 % faster at config 5, from the first pass).
          __builtin_amdgcn_s_setprio(1);
          if constexpr (SCORES) {
            // Weights times 2^kLift2 as fp16, dword 2*c2 + r/2 = rows r, r+1 of
            // column tile 2*half + c2 (k = the lane group's rows); the selector
            // sums dwords 0-1 into row 0 and dwords 2-3 into row 4.
            // Keys at or past the padded end (zero rows, last tile only) get sums
            // too, but no block reads them.
            uint32_t pk[4];
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
              for (int r = 0; r < 4; r += 2) {
                const float p0 = fast_exp2(__builtin_fmaf(sc[c2][r], c, -m[k][r]));
                const float p1 = fast_exp2(__builtin_fmaf(sc[c2][r + 1], c, -m[k][r + 1]));
                pk[2 * c2 + r / 2] = pack_f16(p0, p1);
              }
            __builtin_amdgcn_s_setprio(0);
            colsum[hf] = mfma16x16x32<UKV_DTYPE_F16>(colsel, u32x4{pk[0], pk[1], pk[2], pk[3]}, colsum[hf]);
          } else {
            // Weights of the lane's 8 keys under the column's current max, times
            // 2^kLift1, as fp16: pk[2*c2 + r/2] holds keys r, r+1 of column tile c2.
            // Column tiles at or past the padded end (last tile only) take an
            // addend of -inf, i.e. weight 0.
            uint32_t pk[4];
            bool cvalid[2];
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2) cvalid[c2] = kbase + 16 * (2 * hf + c2) < a.aligned;
            auto weights = [&](float nref) {  // nref = kLift1 - the column's max
#pragma unroll
              for (int c2 = 0; c2 < 2; ++c2) {
                const float add = cvalid[c2] ? nref : -INFINITY;
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                  const float p0 = fast_exp2(__builtin_fmaf(sc[c2][r], c, add));
                  const float p1 = fast_exp2(__builtin_fmaf(sc[c2][r + 1], c, add));
                  pk[2 * c2 + r / 2] = pack_f16(p0, p1);
                }
              }
            };
            weights(m[k][0]);  // pass 1 keeps kLift1 - max here
            // A weight above 2^8 (packed: above 2^15; inf and NaN lie higher, and
            // non-negative fp16 bit patterns order like their values) moves the
            // columns to their exact running max.
            const u16x2 pmax = __builtin_elementwise_max(
                __builtin_elementwise_max(as_u16x2(pk[0]), as_u16x2(pk[1])),
                __builtin_elementwise_max(as_u16x2(pk[2]), as_u16x2(pk[3])));
            if (__any(__builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(pmax, u16x2{0x7800, 0x7800})) != 0u)) {
              float x = sc[0][0];  // column tile 0 is always valid
#pragma unroll
              for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
                for (int r = 0; r < 4; ++r) x = cvalid[c2] ? fmaxf(x, sc[c2][r]) : x;
              x = max_lane_groups(x);
              const float mo = kLift1 - m[k][0];
              const float mn = fmaxf(mo, x * c);
              const float f = fast_exp2(mo - mn);
#pragma unroll
              for (int r = 0; r < 4; ++r) lsum[k][r] *= f;
              m[k][0] = kLift1 - mn;
              weights(m[k][0]);
            }
            // Column sums on the matrix cores: every row of ones x P is the sum.
            __builtin_amdgcn_s_setprio(0);
            lsum[k] = mfma16x16x32<UKV_DTYPE_F16>(ones, u32x4{pk[0], pk[1], pk[2], pk[3]}, lsum[k]);
          }
          // At most two steps' scores in flight: the next step starts here.
          __builtin_amdgcn_sched_barrier(0);
        }
      }

      // The wave's sums go to its first row tile's slot (TW divides the tiles of a
      // q head, so a wave's tiles share one head): lanes 32-63 take lanes 0-31 of
      // colsum[1] (column tiles 2, 3), so lane l holds key l.
      if constexpr (SCORES) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(colsum[0][0]),
                                                         __float_as_uint(colsum[1][0]), false, false);
        if (wv * TW < T) lds.colpart[buf][wv * TW][lane] = __uint_as_float(sw[0]) * kUnlift2;
      }

      // Next tile into the other buffer (last read two tiles ago, before the previous barrier).
      if (ti + 1 < t1) stash(buf ^ 1);
      __syncthreads();  // tile ti+1 and this tile's column sums are visible
      if (ti + 2 < t1) fetch(ti + 2);

    }
    // The tile loop's last column sums (visible after its last barrier).
    if constexpr (SCORES) head_sum(t1 - 1, (t1 - 1 - t0) & 1);

    if constexpr (!SCORES) {
      // This range's partial (m, l) of query row l16 of each tile (lane group 0).
#pragma unroll
      for (int k = 0; k < TW; ++k) {
        const int tile = wv * TW + k;
        if (tile < T && lg == 0) {
          const int row = tile * 16 + l16;
          const int64_t grow = (int64_t)(h0 + row / a.obs) * a.obs + row % a.obs;
          a.part_stats[((int64_t)item * a.S + s) * rows_all + grow] =
              make_float2(kLift1 - m[k][0], lsum[k][0] * (1.f / 128.f));
        }
      }
    }
  }

  if constexpr (SCORES) {
    __syncthreads();
    // Sums over 16-key blocks of the range, divided by obs (the mean over queries).
    const float inv_obs = 1.f / (float)a.obs;
    const int nb = (t1 - t0) * (kSnapTile / 16);
    for (int i = tid; i < nb; i += blockDim.x) {
      const int n = key0 / 16 + i;
      if (n >= a.n_blocks) continue;
      float x = 0.f;
#pragma unroll
      for (int t = 0; t < 16; ++t) x += lds.colmax[16 * i + t];
      a.raw[(int64_t)item * a.n_blocks + n] = x * inv_obs;
    }
  }
}

// (m, l) partials of the S ranges -> m' = m + log2(l) per (item, row), so that
// the weight of a score x (log2 units) is exp2(x - m').
__global__ void __launch_bounds__(256) snap_stats_merge_kernel(const SnapArgs a) {
  const int rows_all = a.Hq * a.obs;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)a.items * rows_all) return;
  const int64_t item = idx / rows_all, row = idx % rows_all;
  if (a.redo && a.redo[item] == 0) return;
  float mx = -INFINITY;
  for (int s = 0; s < a.S; ++s) mx = fmaxf(mx, a.part_stats[(item * a.S + s) * rows_all + row].x);
  float l = 0.f;
  for (int s = 0; s < a.S; ++s) {
    const float2 p = a.part_stats[(item * a.S + s) * rows_all + row];
    l += p.y * fast_exp2(p.x - mx);
  }
  a.stats[idx] = make_float2(mx + log2f(l), 0.f);
}

// Row statistics supplied by the caller (the prefill's observation rows): copied into
// a.stats; an item with a row marked y != 0 (a sum that lost precision) or a non-finite
// one gets redo[item] = 1, so that pass 1 recomputes its rows from the keys.
__global__ void __launch_bounds__(256) snap_stats_import_kernel(const SnapArgs a, const float2* given) {
  const int rows_all = a.Hq * a.obs;
  const int64_t item = blockIdx.x;
  bool bad = false;
  for (int row = threadIdx.x; row < rows_all; row += blockDim.x) {
    const float2 v = given[item * rows_all + row];
    a.stats[item * rows_all + row] = v;
    bad |= v.y != 0.f || !__builtin_isfinite(v.x);
  }
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) a.redo[item] = bad ? 1 : 0;
}

// out[item][n] = max(raw[n-1], raw[n], raw[n+1]) when n_blocks >= 3, else raw[n].
__global__ void __launch_bounds__(256) snap_pool_kernel(const SnapArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)a.items * a.n_blocks) return;
  const int64_t item = idx / a.n_blocks;
  const int n = (int)(idx % a.n_blocks);
  const float* r = a.raw + item * a.n_blocks;
  float x = r[n];
  if (a.n_blocks >= 3) {
    if (n > 0) x = fmaxf(x, r[n - 1]);
    if (n + 1 < a.n_blocks) x = fmaxf(x, r[n + 1]);
  }
  a.out[item * a.out_stride + n] = x;
}

// Scalar path, pass 1: one thread per (item, q head, query): (m, 1/l) over all keys.
template <int DT>
__global__ void __launch_bounds__(256) snap_scalar_stats_kernel(const SnapArgs a) {
  const int rows_all = a.Hq * a.obs;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)a.items * rows_all) return;
  const int item = (int)(idx / rows_all), row = (int)(idx % rows_all);
  if (a.redo && a.redo[item] == 0) return;
  const int h = row / a.obs, i = row % a.obs, g = h / a.n_rep;
  const uint16_t* qp = a.q + (int64_t)item * a.q_si + (int64_t)h * a.q_sh + (int64_t)i * a.q_st;
  float mx = -INFINITY, l = 0.f;
  for (int j = 0; j < a.aligned; ++j) {
    const int64_t off = key_row(a, item, j, g);
    float dot = 0.f;
    if (off >= 0)
      for (int d = 0; d < a.D; ++d) dot += Elem<DT>::one(qp[d]) * Elem<DT>::one(a.k[off + d]);
    const float x = dot * a.scale_log2;
    const float mn = fmaxf(mx, x);
    l = l * fast_exp2(mx - mn) + fast_exp2(x - mn);
    mx = mn;
  }
  a.stats[idx] = make_float2(mx + log2f(l), 0.f);
}

// Scalar path, pass 2: one workgroup per (item, 16-key block): thread t < 16
// owns key 16n + t and loops over every (head, query).
template <int DT>
__global__ void __launch_bounds__(64) snap_scalar_scores_kernel(const SnapArgs a) {
  const int item = blockIdx.y, n = blockIdx.x;
  __shared__ float col[16];
  const int t = threadIdx.x;
  if (t < 16) {
    const int j = 16 * n + t;
    float best = 0.f;
    for (int h = 0; h < a.Hq; ++h) {
      const int g = h / a.n_rep;
      const int64_t off = key_row(a, item, j, g);
      float sum = 0.f;
      for (int i = 0; i < a.obs; ++i) {
        const uint16_t* qp = a.q + (int64_t)item * a.q_si + (int64_t)h * a.q_sh + (int64_t)i * a.q_st;
        float dot = 0.f;
        if (off >= 0)
          for (int d = 0; d < a.D; ++d) dot += Elem<DT>::one(qp[d]) * Elem<DT>::one(a.k[off + d]);
        const float2 st = a.stats[(int64_t)item * a.Hq * a.obs + (int64_t)h * a.obs + i];
        sum += fast_exp2(dot * a.scale_log2 - st.x);
      }
      best = fmaxf(best, sum / (float)a.obs);
    }
    col[t] = best;
  }
  __syncthreads();
  if (t == 0) {
    float x = 0.f;
    for (int u = 0; u < 16; ++u) x += col[u];
    a.raw[(int64_t)item * a.n_blocks + n] = x;
  }
}

namespace {

int snap_cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

struct SnapPlan {
  bool tiled;
  int hp, tw, parts, S, Kt, aligned, n_blocks, L_mid;
  size_t part_off, stats_off, raw_off, redo_off, total;
};

SnapPlan snap_plan(int items, int seq_len, int sink, int obs, int num_q_heads, int n_rep, int head_dim,
                   int block_size, bool aligned_rows) {
  SnapPlan p{};
  p.L_mid = seq_len - sink - obs;
  p.aligned = ((std::max(1, p.L_mid) + block_size - 1) / block_size) * block_size;
  p.n_blocks = p.aligned / block_size;
  p.Kt = (p.aligned + kSnapTile - 1) / kSnapTile;
  // Heads per unit: the largest divisor of n_rep whose row tiles fit the waves
  // with TW tiles each, TW (1, 2 or 4, the smallest that fits) dividing the
  // tiles of one q head, so that a wave's tiles never span two heads.
  p.hp = 0;
  p.tw = 0;
  const int tph = obs / 16;
  if (obs % 16 == 0 && tph > 0)
    for (int h = std::min(n_rep, 32); h >= 1 && p.hp == 0; --h) {
      if (n_rep % h != 0) continue;
      for (int tw = 1; tw <= kSnapMaxTW; tw *= 2)
        if (tph % tw == 0 && h * tph <= kSnapWaves * tw) {
          p.hp = h;
          p.tw = tw;
          break;
        }
    }
  p.tiled = (head_dim == 64 || head_dim == 128) && p.hp > 0 && aligned_rows;
  p.parts = p.tiled ? n_rep / p.hp : 1;
  if (p.tiled) {
    const int want = (2 * snap_cu_count() + items - 1) / std::max(1, items);
    const int need = (p.Kt * kSnapTile + kSnapMaxKeys - 1) / kSnapMaxKeys;
    p.S = std::max(need, std::min(want, std::max(1, p.Kt / 4)));
    p.S = std::min(p.S, p.Kt);
  } else {
    p.S = 1;
  }
  const size_t rows_all = (size_t)num_q_heads * obs;
  p.part_off = 0;
  p.stats_off = a256((size_t)items * p.S * rows_all * sizeof(float2));
  p.raw_off = p.stats_off + a256((size_t)items * rows_all * sizeof(float2));
  p.redo_off = p.raw_off + a256((size_t)items * p.n_blocks * sizeof(float));
  p.total = p.redo_off + a256((size_t)items * sizeof(int32_t));
  return p;
}

// With a.redo set, pass 1 and the merge skip the items whose statistics were imported.
template <int DT, int D, int TW>
void launch_tiled(const SnapArgs& a, const SnapPlan& p, hipStream_t st) {
  const int64_t rows = (int64_t)a.items * a.Hq * a.obs;
  const dim3 grid(p.S, a.items);
  hipLaunchKernelGGL((snap_tile_kernel<DT, D, false, TW>), grid, dim3(64 * kSnapWaves), 0, st, a);
  hipLaunchKernelGGL(snap_stats_merge_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, a);
  hipLaunchKernelGGL((snap_tile_kernel<DT, D, true, TW>), grid, dim3(64 * kSnapWaves), 0, st, a);
}

template <int DT, int D>
void launch_tiled_tw(const SnapArgs& a, const SnapPlan& p, hipStream_t st) {
  if (p.tw == 1)
    launch_tiled<DT, D, 1>(a, p, st);
  else if (p.tw == 2)
    launch_tiled<DT, D, 2>(a, p, st);
  else
    launch_tiled<DT, D, 4>(a, p, st);
}

template <int DT>
void launch_snap(const SnapArgs& a, const SnapPlan& p, hipStream_t st, const float2* given) {
  if (given)
    hipLaunchKernelGGL(snap_stats_import_kernel, dim3((unsigned)a.items), dim3(256), 0, st, a, given);
  if (p.tiled) {
    if (a.D == 64)
      launch_tiled_tw<DT, 64>(a, p, st);
    else
      launch_tiled_tw<DT, 128>(a, p, st);
  } else {
    const int64_t rows = (int64_t)a.items * a.Hq * a.obs;
    hipLaunchKernelGGL(snap_scalar_stats_kernel<DT>, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, a);
    hipLaunchKernelGGL(snap_scalar_scores_kernel<DT>, dim3(a.n_blocks, a.items), dim3(64), 0, st, a);
  }
  const int64_t nout = (int64_t)a.items * a.n_blocks;
  hipLaunchKernelGGL(snap_pool_kernel, dim3((unsigned)((nout + 255) / 256)), dim3(256), 0, st, a);
}

bool snap_aligned(const void* q, const void* k, const int64_t* qs, const int64_t* ks) {
  auto m8 = [](int64_t x) { return (x & 7) == 0; };
  return (reinterpret_cast<uintptr_t>(q) & 15u) == 0 && (reinterpret_cast<uintptr_t>(k) & 15u) == 0 && m8(qs[0]) &&
         m8(qs[1]) && m8(qs[2]) && m8(ks[0]) && m8(ks[1]) && m8(ks[2]) && m8(ks[3]);
}

bool snap_shape_ok(int layers, int seqs, int seq_len, int sink, int obs, int num_q_heads, int num_kv_heads,
                   int head_dim, int n_rep, int block_size) {
  // Blocks are the pool's 16-token pages (the kernels sum scores over 16 keys).
  return layers > 0 && seqs > 0 && seq_len > 0 && sink >= 0 && obs > 0 && num_q_heads > 0 && num_kv_heads > 0 &&
         head_dim > 0 && n_rep > 0 && block_size == 16 && num_q_heads == num_kv_heads * n_rep;
}

}  // namespace
}  // namespace ukv

using namespace ukv;

extern "C" int ukv_snapkv_block_count(int seq_len, int sink_len, int obs_len, int block_size) {
  if (block_size <= 0 || seq_len < sink_len + obs_len + block_size) return 0;
  const int L_mid = seq_len - sink_len - obs_len;
  return (std::max(1, L_mid) + block_size - 1) / block_size;
}

extern "C" size_t ukv_snapkv_workspace_bytes(int layers, int seqs, int seq_len, int sink_len, int obs_len,
                                             int num_q_heads, int num_kv_heads, int head_dim, int n_rep,
                                             int block_size) {
  if (!snap_shape_ok(layers, seqs, seq_len, sink_len, obs_len, num_q_heads, num_kv_heads, head_dim, n_rep,
                     block_size) ||
      ukv_snapkv_block_count(seq_len, sink_len, obs_len, block_size) == 0)
    return 0;
  // The tiled plan needs at least as much as the scalar one; size for the larger.
  return snap_plan(layers * seqs, seq_len, sink_len, obs_len, num_q_heads, n_rep, head_dim, block_size, true).total;
}

namespace {

int snapkv_scores_impl(const void* q_obs, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                       const int32_t* block_table, int max_blocks, int num_pages, int layers, int seqs, int seq_len,
                       int sink_len, int obs_len, int num_q_heads, int num_kv_heads, int head_dim, int n_rep,
                       int block_size, float softmax_scale, int dtype, const float* given_stats, float* scores,
                       int64_t scores_stride, void* workspace, size_t workspace_bytes, ukv_stream_t stream) {
  if (!snap_shape_ok(layers, seqs, seq_len, sink_len, obs_len, num_q_heads, num_kv_heads, head_dim, n_rep,
                     block_size))
    return UKV_ERR_INVALID_ARGUMENT;
  if (dtype != UKV_DTYPE_F16 && dtype != UKV_DTYPE_BF16) return UKV_ERR_DTYPE;
  const int n_blocks = ukv_snapkv_block_count(seq_len, sink_len, obs_len, block_size);
  if (n_blocks == 0) return UKV_OK;  // too short: no middle blocks to score (the reference's empty result)
  if (!q_obs || !q_strides || !k || !k_strides || !scores || scores_stride < n_blocks) return UKV_ERR_INVALID_ARGUMENT;
  if (block_table && (max_blocks <= 0 || num_pages <= 0)) return UKV_ERR_INVALID_ARGUMENT;
  if ((int64_t)layers * seqs > 65535) return UKV_ERR_INVALID_ARGUMENT;
  const int items = layers * seqs;
  const SnapPlan p = snap_plan(items, seq_len, sink_len, obs_len, num_q_heads, n_rep, head_dim, block_size,
                               snap_aligned(q_obs, k, q_strides, k_strides));
  if (!workspace || workspace_bytes < p.total || (reinterpret_cast<uintptr_t>(workspace) & 15u)) return UKV_ERR_WORKSPACE;

  SnapArgs a{};
  a.q = static_cast<const uint16_t*>(q_obs);
  a.q_si = q_strides[0];
  a.q_sh = q_strides[1];
  a.q_st = q_strides[2];
  a.k = static_cast<const uint16_t*>(k);
  a.k_sl = k_strides[0];
  a.k_sb = k_strides[1];
  a.k_st = k_strides[2];
  a.k_sh = k_strides[3];
  a.table = block_table;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.layers = layers;
  a.items = items;
  a.sink = sink_len;
  a.obs = obs_len;
  a.L_mid = p.L_mid;
  a.aligned = p.aligned;
  a.n_blocks = p.n_blocks;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.n_rep = n_rep;
  a.D = head_dim;
  a.hp = p.hp;
  a.parts = p.parts;
  a.S = p.S;
  a.Kt = p.Kt;
  a.scale_log2 = softmax_scale * kLog2e;
  char* ws = static_cast<char*>(workspace);
  a.part_stats = reinterpret_cast<float2*>(ws + p.part_off);
  a.stats = reinterpret_cast<float2*>(ws + p.stats_off);
  a.raw = reinterpret_cast<float*>(ws + p.raw_off);
  a.redo = given_stats ? reinterpret_cast<int32_t*>(ws + p.redo_off) : nullptr;
  a.out = scores;
  a.out_stride = scores_stride;
  const float2* given = reinterpret_cast<const float2*>(given_stats);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == UKV_DTYPE_BF16)
    launch_snap<UKV_DTYPE_BF16>(a, p, st, given);
  else
    launch_snap<UKV_DTYPE_F16>(a, p, st, given);
  return hipGetLastError() == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}

}  // namespace

extern "C" int ukv_snapkv_scores(const void* q_obs, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                 const int32_t* block_table, int max_blocks, int num_pages, int layers, int seqs,
                                 int seq_len, int sink_len, int obs_len, int num_q_heads, int num_kv_heads,
                                 int head_dim, int n_rep, int block_size, float softmax_scale, int dtype,
                                 float* scores, int64_t scores_stride, void* workspace, size_t workspace_bytes,
                                 ukv_stream_t stream) {
  return snapkv_scores_impl(q_obs, q_strides, k, k_strides, block_table, max_blocks, num_pages, layers, seqs,
                            seq_len, sink_len, obs_len, num_q_heads, num_kv_heads, head_dim, n_rep, block_size,
                            softmax_scale, dtype, nullptr, scores, scores_stride, workspace, workspace_bytes,
                            stream);
}

extern "C" int ukv_snapkv_scores_from_stats(const void* q_obs, const int64_t* q_strides, const void* k,
                                            const int64_t* k_strides, const int32_t* block_table, int max_blocks,
                                            int num_pages, int layers, int seqs, int seq_len, int sink_len,
                                            int obs_len, int num_q_heads, int num_kv_heads, int head_dim, int n_rep,
                                            int block_size, float softmax_scale, int dtype, const float* obs_stats,
                                            float* scores, int64_t scores_stride, void* workspace,
                                            size_t workspace_bytes, ukv_stream_t stream) {
  if (!obs_stats || (reinterpret_cast<uintptr_t>(obs_stats) & 7u)) return UKV_ERR_INVALID_ARGUMENT;
  return snapkv_scores_impl(q_obs, q_strides, k, k_strides, block_table, max_blocks, num_pages, layers, seqs,
                            seq_len, sink_len, obs_len, num_q_heads, num_kv_heads, head_dim, n_rep, block_size,
                            softmax_scale, dtype, obs_stats, scores, scores_stride, workspace, workspace_bytes,
                            stream);
}
