// Element steps of the attention prologue, shared by the one-pass prologue
// kernel (qk_prologue.hip) and the neighbourhood-attention kernels that
// prepare q as they load it (na3d_fwd.hip), so both round at the same points:
//   norm:  bf16( bf16(x * rinv) * bf16(w) ),  rinv = 1 / sqrt(mean(x^2) + eps)
//   scale: bf16( y * bf16(post_scale) )
//   rope:  (y1, y2) -> (bf16(y1 c - y2 s), bf16(y2 c + y1 s)) in fp32
#pragma once

#include "vx_gfx950.hpp"

namespace vx {

__device__ __forceinline__ float rsqrt_ieee(float x) { return 1.0f / __builtin_sqrtf(x); }

// 1 / sqrt(sum_sq / n + eps), as the reference's RMSNorm (fp32 statistics).
__device__ __forceinline__ float rms_inv(float sum_sq, int n, float eps) {
#pragma clang fp contract(off)
  return rsqrt_ieee(sum_sq / (float)n + eps);
}

__device__ __forceinline__ bf16 rms_elem(float x, float rinv, float w) {
#pragma clang fp contract(off)
  const float n = (float)(bf16)(x * rinv);
  return (bf16)(n * (float)(bf16)w);
}

// ps is bf16(post_scale) held in fp32
__device__ __forceinline__ bf16 scale_elem(float y, float ps) { return (bf16)(y * ps); }

// rotates the pair (v[2p], v[2p+1]); products and difference rounded
// separately (no fused multiply-add), so every kernel that inlines this
// rounds the same way
__device__ __forceinline__ void rope_pair(bf16x8& v, int p, float c, float s) {
#pragma clang fp contract(off)
  const float x1 = (float)v[2 * p], x2 = (float)v[2 * p + 1];
  v[2 * p] = (bf16)(x1 * c - x2 * s);
  v[2 * p + 1] = (bf16)(x2 * c + x1 * s);
}

// Sum of squares of 8 bf16 values (fp32, in element order).
__device__ __forceinline__ float sum_sq8(const bf16x8& v) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = __builtin_fmaf((float)v[e], (float)v[e], s);
  return s;
}

}  // namespace vx
