// gfx950 (CDNA4) building blocks shared by the attention kernels: vector
// types, the bf16 MFMA, the LDS transpose read, cross-half lane exchange and
// the exp2 used by the softmax.
//
// MFMA v_mfma_f32_32x32x16_bf16 register layouts (lane l of a wave64):
//   A (32 x 16, row-major M x K): lane l holds row l%32, k = (l/32)*8 + 0..7
//   B (16 x 32, K x N):           lane l holds col l%32, k = (l/32)*8 + 0..7
//   C (32 x 32):                  lane l holds col l%32, element i (0..15) is
//                                 row (i/4)*8 + (l/32)*4 + i%4
// ds_read_b64_tr_b16 (per group of 16 lanes): lane 4r+c supplies the address
// of row r, columns 4c..4c+3 of a 4 x 16 block of 16-bit elements; lane i of
// the group receives column i of rows 0..3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vx {

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define VX_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 2^x on the hardware transcendental unit (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value of x held by lane l^32 combined with lane l's own: returns the pair
// {x[l%32], x[l%32 + 32]} in every lane (one v_permlane32_swap).
__device__ __forceinline__ void halves(float x, float& lo, float& hi) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
__device__ __forceinline__ float halves_max(float x) {
  float lo, hi;
  halves(x, lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float halves_sum(float x) {
  float lo, hi;
  halves(x, lo, hi);
  return lo + hi;
}

__device__ __forceinline__ bf16x4 lds_read_tr16(const unsigned char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p));
  return __builtin_bit_cast(bf16x4, r);
}

__device__ __forceinline__ bf16x8 concat(bf16x4 a, bf16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Sum of eight bf16 values accumulated into fp32 (four v_dot2_f32_bf16).
__device__ __forceinline__ float sum8(bf16x8 p, float acc) {
  const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 0, 1), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 2, 3), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 4, 5), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 6, 7), one, acc, false);
  return acc;
}

}  // namespace vx
