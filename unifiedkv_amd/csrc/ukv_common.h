// Shared device helpers for the gfx950 (CDNA4) kernels of the Page16 hot path.
//
// Everything here is written for wave64 and the gfx950 instruction set only:
// 16-byte global loads, DPP row reductions inside a 16-lane row, and the
// double-rate 16x16x32 MFMA builtins.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ukv.h"

namespace ukv {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr float kNegFltMax = -3.4028234663852886e38f;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Element conversions. A 32-bit word holds two 16-bit elements, low half first.
// ---------------------------------------------------------------------------
template <int DT> struct Elem;

template <> struct Elem<UKV_DTYPE_BF16> {
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static __device__ __forceinline__ float one(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
  // fp32 -> bf16 with round-to-nearest-even; NaN stays a quiet NaN.
  static __device__ __forceinline__ uint16_t from_float(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
  }
};

template <> struct Elem<UKV_DTYPE_F16> {
  static __device__ __forceinline__ float lo(uint32_t w) {
    return float(__builtin_bit_cast(_Float16, uint16_t(w & 0xffffu)));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16)));
  }
  static __device__ __forceinline__ float one(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }
  static __device__ __forceinline__ uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, _Float16(f));
  }
};

// D(16x16, fp32) += A(16x32) * B(32x16) on packed 16-bit operands (8 per lane).
template <int DT> __device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);

template <> __device__ __forceinline__ f32x4 mfma16x16x32<UKV_DTYPE_BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma16x16x32<UKV_DTYPE_F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// D(16x16, fp32) += A(16x16) * B(16x16) on packed 16-bit operands (4 per lane).
template <int DT> __device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c);

template <> __device__ __forceinline__ f32x4 mfma16x16x16<UKV_DTYPE_BF16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                   0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma16x16x16<UKV_DTYPE_F16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                               0);
}

// ---------------------------------------------------------------------------
// Row (16-lane) reductions with DPP. After the four steps every lane of the
// row holds the reduction over all 16 lanes of its row.
//   0xB1 = quad_perm [1,0,3,2]   0x4E = quad_perm [2,3,0,1]
//   0x141 = row_half_mirror      0x140 = row_mirror
// ---------------------------------------------------------------------------
#define UKV_DPP(x, ctrl) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), (ctrl), 0xf, 0xf, false))

__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, UKV_DPP(x, 0xB1));
  x = fmaxf(x, UKV_DPP(x, 0x4E));
  x = fmaxf(x, UKV_DPP(x, 0x141));
  x = fmaxf(x, UKV_DPP(x, 0x140));
  return x;
}

__device__ __forceinline__ float row_sum16(float x) {
  x += UKV_DPP(x, 0xB1);
  x += UKV_DPP(x, 0x4E);
  x += UKV_DPP(x, 0x141);
  x += UKV_DPP(x, 0x140);
  return x;
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two floats -> two packed 16-bit values (round to nearest even).
__device__ __forceinline__ uint32_t pack_f16(float x0, float x1) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, f16x2));
}
__device__ __forceinline__ uint32_t pack_bf16(float x0, float x1) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, bf16x2));
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 as_u16x2(uint32_t w) { return __builtin_bit_cast(u16x2, w); }

// Host side, page_ops.hip: writes row b of k_new/v_new ([batch][num_heads][head_dim],
// strides new_strides[0..1]) at position lens[b] + pos_offset of sequence b (page
// block_table[b][pos / block_size], slot pos % block_size); positions outside the table
// and invalid page ids are skipped. new_lens (nullable) receives lens + 1.
int append_decode_rows(void* k_pool_layer, void* v_pool_layer, const int64_t* k_strides, const int64_t* v_strides,
                       const void* k_new, const void* v_new, const int64_t* new_strides, const int32_t* block_table,
                       int max_blocks, const int32_t* lens, int pos_offset, int32_t* new_lens, int batch,
                       int block_size, int num_heads, int head_dim, int num_pages, ukv_stream_t stream);

}  // namespace ukv
