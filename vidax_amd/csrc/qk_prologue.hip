// Fused attention prologue for gfx950: RMSNorm of q or k (over the whole
// projected row or per head) followed by the 3D rotary embedding, in one pass
// over HBM (read the bf16 row once, write the bf16 result once).
//
// Per token row x (n_heads * head_dim bf16 values, one wave per row):
//   norm:  y = bf16( bf16(x * rsqrt(mean(x^2) + eps)) * bf16(w) )
//          mean over the whole row (group = row) or over each head (group =
//          head_dim); fp32 statistics. Skipped when no weight is given.
//   scale: y = bf16(y * bf16(post_scale)), skipped when post_scale is 1
//          (the neighbourhood-attention block's q * head_dim^-0.5).
//   rope:  adjacent pairs (y[2j], y[2j+1]) of every head are rotated by the
//          token's (cos[j], sin[j]) in fp32 and rounded to bf16. Skipped when
//          no tables are given.
// These are the dtype points of the reference's RMSNorm (normalise in fp32,
// cast, multiply by the cast weight), a bf16 array times a weakly typed
// scalar, and the fp32 rotations of apply_rope3d / _apply_abs_rope (cast back).
//
// Layout: row s of batch b starts at x + b*x_bstride + s*x_sstride (elements)
// and is contiguous; lane l of the wave owns the 16-byte chunks l, l + 64, ...
// of the row, so every load and store is one coalesced 1 KiB wave access.
#include "vx_gfx950.hpp"
#include "vx_kernels.h"
#include "vx_qk_prep.hpp"

#include <string>

namespace vx {
namespace {

constexpr int kWavesPerBlock = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over aligned groups of n lanes (n = head_dim / 8: the lanes whose
// chunks make up one head in the same iteration; n divides 64).
__device__ __forceinline__ float group_sum(float v, int n) {
  for (int off = n >> 1; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ bf16 to_bf16(float x) { return (bf16)x; }

// NCHUNK: 16-byte chunks per lane (exact); FULL: the row is a whole number of
// 1 KiB wave accesses, so no lane is ever idle and no chunk needs a bounds test.
template <int NCHUNK, bool FULL>
__global__ __launch_bounds__(kWavesPerBlock * 64) void qk_prologue_kernel(const PrologueArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.S) return;  // whole waves only
  const int b = (int)(row / a.S);
  const int s = (int)(row - (int64_t)b * a.S);
  const int row_len = a.H * a.D;
  const int n_chunks = row_len / 8;
  auto live = [&](int c) { return FULL || c < n_chunks; };
  const bf16* xr = (const bf16*)a.x + b * a.x_bstride + s * a.x_sstride;
  bf16* orow = (bf16*)a.out + b * a.o_bstride + s * a.o_sstride;

  bf16x8 v[NCHUNK];
  float ss[NCHUNK];
#pragma unroll
  for (int i = 0; i < NCHUNK; ++i) {
    const int c = lane + 64 * i;
    ss[i] = 0.f;
    if (live(c)) {
      v[i] = __builtin_nontemporal_load((const bf16x8*)(xr + c * 8));  // read once: streaming
      ss[i] = sum_sq8(v[i]);
    }
  }

  if (a.weight != nullptr) {
    float rinv_row = 0.f;
    if (!a.per_head) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < NCHUNK; ++i) t += ss[i];
      rinv_row = rms_inv(wave_sum(t), row_len, a.eps);
    }
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int c = lane + 64 * i;
      // per head: the head_dim / 8 lanes of an aligned group share a head
      float rinv = rinv_row;
      if (a.per_head) rinv = rms_inv(group_sum(ss[i], a.D / 8), a.D, a.eps);
      if (live(c)) {
        const f32x4 w0 = *(const f32x4*)(a.weight + c * 8);
        const f32x4 w1 = *(const f32x4*)(a.weight + c * 8 + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = rms_elem((float)v[i][e], rinv, e < 4 ? w0[e] : w1[e - 4]);
      }
    }
  }

  if (a.post_scale != 1.0f) {
    const float ps = (float)to_bf16(a.post_scale);
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      if (live(lane + 64 * i)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = scale_elem((float)v[i][e], ps);
      }
    }
  }

  if (a.cos != nullptr) {
    const float* cr = a.cos + (int64_t)s * a.tab_stride;
    const float* sr = a.sin + (int64_t)s * a.tab_stride;
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int c = lane + 64 * i;
      if (live(c)) {
        const int j0 = ((c * 8) % a.D) / 2;  // first pair of the chunk within its head
        const f32x4 cs = *(const f32x4*)(cr + j0);
        const f32x4 sn = *(const f32x4*)(sr + j0);
#pragma unroll
        for (int p = 0; p < 4; ++p) rope_pair(v[i], p, cs[p], sn[p]);
      }
    }
  }

#pragma unroll
  for (int i = 0; i < NCHUNK; ++i) {
    const int c = lane + 64 * i;
    if (live(c)) __builtin_nontemporal_store(v[i], (bf16x8*)(orow + c * 8));  // written once
  }
}

template <int NCHUNK, bool FULL>
const char* prologue_kernel_name() {
  static const std::string name =
      "qk_prologue_kernel<" + std::to_string(NCHUNK) + ", " + (FULL ? "true" : "false") + ">";
  return name.c_str();
}

template <int NCHUNK>
int launch(const PrologueArgs& a, hipStream_t st, const char** launched) {
  const int64_t rows = (int64_t)a.B * a.S;
  dim3 grid((unsigned)((rows + kWavesPerBlock - 1) / kWavesPerBlock));
  if ((a.H * a.D) % 512 == 0) {
    hipLaunchKernelGGL((qk_prologue_kernel<NCHUNK, true>), grid, dim3(kWavesPerBlock * 64), 0, st, a);
    *launched = prologue_kernel_name<NCHUNK, true>();
  } else {
    hipLaunchKernelGGL((qk_prologue_kernel<NCHUNK, false>), grid, dim3(kWavesPerBlock * 64), 0, st, a);
    *launched = prologue_kernel_name<NCHUNK, false>();
  }
  return (int)hipGetLastError();
}

}  // namespace

int launch_qk_prologue(const PrologueArgs& a, void* stream, const char** launched) {
  hipStream_t st = (hipStream_t)stream;
  switch ((a.H * a.D / 8 + 63) / 64) {  // chunks per lane
    case 1: return launch<1>(a, st, launched);
    case 2: return launch<2>(a, st, launched);
    case 3: return launch<3>(a, st, launched);
    case 4: return launch<4>(a, st, launched);
    case 5: return launch<5>(a, st, launched);
    case 6: return launch<6>(a, st, launched);
    case 7: return launch<7>(a, st, launched);
    case 8: return launch<8>(a, st, launched);
    case 9: return launch<9>(a, st, launched);
    case 10: return launch<10>(a, st, launched);
    case 11: return launch<11>(a, st, launched);
    case 12: return launch<12>(a, st, launched);
    case 13: return launch<13>(a, st, launched);
    case 14: return launch<14>(a, st, launched);
    case 15: return launch<15>(a, st, launched);
    case 16: return launch<16>(a, st, launched);
    default: return (int)hipErrorNotSupported;
  }
}

}  // namespace vx
