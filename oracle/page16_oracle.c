/*
 * TEST INFRASTRUCTURE ONLY - the CPU oracle of the Page16 hot path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / reported CPU baseline. The
 * product (libukv.so) never links or calls it.
 *
 * Restates the reference's Page16 decode program (BP-KV
 * core/page16_native.py:34-80) in plain C, fp32, in the reference's order:
 *   q load            :40-44   q_f32[d] = q[(b*Hq + h)*D + d]
 *   kv head           :36      kv_h = h / n_rep
 *   running state     :47-49   m = -FLT_MAX, l = 0, acc[:] = 0
 *   page loop         :52-53   blk = 0 .. max_blocks-1 (every table column)
 *   token mask        :54-55   token = blk*16 + t valid iff token < seq_len
 *   page id           :56      bid = block_table[b*max_blocks + blk]
 *   scores            :57-60   s_t = (sum_d K[bid,t,kv_h,d]*q[d]) * scale,
 *                              masked -> -FLT_MAX (masked K loads are 0)
 *   online softmax    :62-67   m' = max(m, max_t s_t); alpha = exp(m - m');
 *                              p_t = exp(s_t - m') (0 if masked);
 *                              l = l*alpha + sum_t p_t
 *   P.V               :68-70   acc = acc*alpha + sum_t p_t*V[bid,t,kv_h,:]
 *   output            :75-80   out = acc / l   (rounded to q's dtype by caller)
 * One documented deviation: a page id outside [0, num_pages) of a page that
 * holds valid tokens is UB in the reference (an out-of-bounds read); here, as
 * in libukv.so, such a page's tokens are treated as masked.
 *
 * `mutation` plants a known mistake for the oracle's own discrimination tests
 * (0 = faithful restatement; see the switch below).
 */
#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define NEG_FLT_MAX (-3.4028234663852886e38f)

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: renormalise */
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while ((man & 0x400u) == 0);
      u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 0x1f) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float load_elem(const uint16_t* p, int dtype) { return dtype == 1 ? bf16_to_f32(*p) : f16_to_f32(*p); }

/* Element -> fp32 for a whole buffer (used by the Python side for inputs). */
/* Threads of the OpenMP page loop (the CPU baseline reports all-core and 1-thread figures). */
void ukvo_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}

void ukvo_to_f32(const uint16_t* src, float* dst, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) dst[i] = load_elem(src + i, dtype);
}

/*
 * q [B][Hq][D], k/v [num_pages][16][Hkv][D] (contiguous, dtype 0=f16 1=bf16),
 * block_table int32 [B][max_blocks], seqlens int32 [B], out fp32 [B][Hq][D].
 * Returns 0, or -1 on an argument the reference would reject.
 */
int ukvo_page16_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* block_table,
                       const int32_t* seqlens, float* out, int B, int Hq, int Hkv, int D, int n_rep,
                       int max_blocks, int num_pages, float scale, int dtype, int mutation) {
  if (B <= 0 || Hq <= 0 || D <= 0 || Hkv <= 0 || n_rep <= 0 || D > 256) return -1;
  const int64_t tok_stride = (int64_t)Hkv * D;
  const int64_t page_stride = 16 * tok_stride;

#pragma omp parallel for schedule(dynamic, 1)
  for (int bh = 0; bh < B * Hq; ++bh) {
    const int b = bh / Hq;
    const int h = bh % Hq;
    int kv_h = h / n_rep;
    if (mutation == 1) kv_h = h % Hkv; /* wrong GQA map */
    float qf[256], acc[256];
    for (int d = 0; d < D; ++d) {
      qf[d] = load_elem(q + ((int64_t)b * Hq + h) * D + d, dtype);
      acc[d] = 0.f;
    }
    const int seq_len = seqlens[b];
    float m = NEG_FLT_MAX, l = 0.f;
    for (int blk = 0; blk < max_blocks; ++blk) {
      int bid = block_table[(int64_t)b * max_blocks + blk];
      const int page_ok = bid >= 0 && bid < num_pages;
      float s[16];
      int valid[16];
      float smax = NEG_FLT_MAX;
      for (int t = 0; t < 16; ++t) {
        const int token = blk * 16 + t;
        valid[t] = page_ok && (mutation == 3 ? token <= seq_len : token < seq_len); /* 3: off by one */
        if (valid[t]) {
          const uint16_t* krow;
          if (mutation == 4) /* token and head strides swapped */
            krow = k + (int64_t)bid * page_stride + (int64_t)kv_h * (16 * D) + (int64_t)t * D;
          else
            krow = k + (int64_t)bid * page_stride + (int64_t)t * tok_stride + (int64_t)kv_h * D;
          float dot = 0.f;
          for (int d = 0; d < D; ++d) dot += load_elem(krow + d, dtype) * qf[d];
          s[t] = mutation == 5 ? dot : dot * scale; /* 5: scale dropped */
        } else {
          s[t] = NEG_FLT_MAX;
        }
        if (s[t] > smax) smax = s[t];
      }
      const float m_new = m > smax ? m : smax;
      const float alpha = mutation == 2 ? 1.f : expf(m - m_new); /* 2: no rescale */
      float psum = 0.f;
      float p[16];
      for (int t = 0; t < 16; ++t) {
        p[t] = valid[t] ? expf(s[t] - m_new) : 0.f;
        psum += p[t];
      }
      l = l * alpha + psum;
      float pv[256];
      for (int d = 0; d < D; ++d) pv[d] = 0.f;
      for (int t = 0; t < 16; ++t) { /* per dim: sum over t in token order */
        if (!valid[t]) continue;
        const uint16_t* vrow = v + (int64_t)bid * page_stride + (int64_t)t * tok_stride + (int64_t)kv_h * D;
        for (int d = 0; d < D; ++d) pv[d] += p[t] * load_elem(vrow + d, dtype);
      }
      for (int d = 0; d < D; ++d) acc[d] = acc[d] * alpha + pv[d];
      m = m_new;
    }
    float* o = out + ((int64_t)b * Hq + h) * D;
    for (int d = 0; d < D; ++d) o[d] = acc[d] / l;
  }
  return 0;
}
