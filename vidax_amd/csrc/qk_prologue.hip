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

#include <algorithm>
#include <atomic>
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
//
// Wave w of the grid (n_waves in all) takes rows w, w + n_waves, ... (one
// resident round of waves, consecutive waves on consecutive rows). Across
// its rows a wave keeps the weights of its chunks in registers, rounded to
// bf16 (the rounding rms_elem applies to them), and reads each row's
// rotation table once per lane: a lane's chunks c = lane + 64 i all sit at
// the same position (8 lane) mod head_dim of their heads, since 64 chunks
// span a whole number of heads. With kPrefetch the next row's loads are
// issued before the current row is normalised, rotated and stored, after
// that row's table loads, so that waiting for the tables leaves the next row
// in flight.
// PER_HEAD: the norm is taken per head (a.per_head), whose weight vector of
// head_dim values then gives every chunk of a lane the same 8 weights.
template <int NCHUNK, bool FULL, bool PER_HEAD>
__global__ __launch_bounds__(kWavesPerBlock * 64) void qk_prologue_kernel(const PrologueArgs a) {
  // The next row's loads are issued early (two row buffers) for whole-row
  // norms of up to 10 chunks per lane; the per-head norm (more work per row:
  // one reduction per head) and longer rows keep one buffer and more waves
  // per SIMD.
  constexpr bool kPrefetch = !PER_HEAD && NCHUNK <= 10;
  const int lane = threadIdx.x & 63;
  const int64_t rows = (int64_t)a.B * a.S;
  const int64_t n_waves = (int64_t)gridDim.x * kWavesPerBlock;
  const int64_t r0 = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (r0 >= rows) return;  // whole waves only
  const int row_len = a.H * a.D;
  const int n_chunks = row_len / 8;
  auto live = [&](int c) { return FULL || c < n_chunks; };
  const bool norm = a.weight != nullptr, rope = a.cos != nullptr;
  const int hpos = (lane * 8) % a.D;  // position of this lane's chunks within their heads

  constexpr int kW = PER_HEAD ? 1 : NCHUNK;  // weight chunks held
  bf16x8 wb[kW];
  if (norm) {
#pragma unroll
    for (int i = 0; i < kW; ++i) {
      const int c = lane + 64 * i;
      if (PER_HEAD || live(c)) {
        const float* wp = a.weight + (PER_HEAD ? hpos : c * 8);
        const f32x4 w0 = *(const f32x4*)wp, w1 = *(const f32x4*)(wp + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) wb[i][e] = to_bf16(e < 4 ? w0[e] : w1[e - 4]);
      }
    }
  }
  const float ps = (float)to_bf16(a.post_scale);

  auto row_bs = [&](int64_t r, int& b, int& s) {
    b = (int)(r / a.S);
    s = (int)(r - (int64_t)b * a.S);
  };
  auto load_row = [&](int64_t r, bf16x8 (&v)[NCHUNK]) __attribute__((always_inline)) {
    int b, s;
    row_bs(r, b, s);
    const bf16* xr = (const bf16*)a.x + b * a.x_bstride + s * a.x_sstride;
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int c = lane + 64 * i;
      if (live(c)) v[i] = __builtin_nontemporal_load((const bf16x8*)(xr + c * 8));  // read once: streaming
    }
  };
  // row r, whose x is in v: table loads, then the next row's x (into vn),
  // then the norm, scale and rotation of v and its store
  auto process = [&](int64_t r, bf16x8 (&v)[NCHUNK], int64_t r_next, bf16x8 (&vn)[NCHUNK]) __attribute__((always_inline)) {
    int b, s;
    row_bs(r, b, s);
    f32x4 cs = {}, sn = {};
    if (rope) {
      cs = *(const f32x4*)(a.cos + (int64_t)s * a.tab_stride + hpos / 2);
      sn = *(const f32x4*)(a.sin + (int64_t)s * a.tab_stride + hpos / 2);
    }
    if (r_next < rows) load_row(r_next, vn);
    float ss[NCHUNK];
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) ss[i] = live(lane + 64 * i) ? sum_sq8(v[i]) : 0.f;
    if (norm) {
      float rinv_row = 0.f;
      if (!PER_HEAD) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < NCHUNK; ++i) t += ss[i];
        rinv_row = rms_inv(wave_sum(t), row_len, a.eps);
      }
#pragma unroll
      for (int i = 0; i < NCHUNK; ++i) {
        // per head: the head_dim / 8 lanes of an aligned group share a head
        float rinv = rinv_row;
        if (PER_HEAD) rinv = rms_inv(group_sum(ss[i], a.D / 8), a.D, a.eps);
        if (live(lane + 64 * i)) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[i][e] = rms_elem((float)v[i][e], rinv, (float)wb[PER_HEAD ? 0 : i][e]);
        }
      }
    }
    if (a.post_scale != 1.0f) {
#pragma unroll
      for (int i = 0; i < NCHUNK; ++i) {
        if (live(lane + 64 * i)) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[i][e] = scale_elem((float)v[i][e], ps);
        }
      }
    }
    if (rope) {
#pragma unroll
      for (int i = 0; i < NCHUNK; ++i) {
        if (live(lane + 64 * i)) {
#pragma unroll
          for (int p = 0; p < 4; ++p) rope_pair(v[i], p, cs[p], sn[p]);
        }
      }
    }
    bf16* orow = (bf16*)a.out + b * a.o_bstride + s * a.o_sstride;
#pragma unroll
    for (int i = 0; i < NCHUNK; ++i) {
      const int c = lane + 64 * i;
      if (live(c)) __builtin_nontemporal_store(v[i], (bf16x8*)(orow + c * 8));  // written once
    }
  };

  bf16x8 va[NCHUNK];
  if constexpr (kPrefetch) {
    bf16x8 vb[NCHUNK];
    load_row(r0, va);
    for (int64_t r = r0; r < rows; r += 2 * n_waves) {
      process(r, va, r + n_waves, vb);
      if (r + n_waves < rows) process(r + n_waves, vb, r + 2 * n_waves, va);
    }
  } else {
    for (int64_t r = r0; r < rows; r += n_waves) {
      load_row(r, va);
      process(r, va, rows, va);
    }
  }
}

template <int NCHUNK, bool FULL, bool PER_HEAD>
const char* prologue_kernel_name() {
  static const std::string name = "qk_prologue_kernel<" + std::to_string(NCHUNK) + ", " + (FULL ? "true" : "false") +
                                  ", " + (PER_HEAD ? "true" : "false") + ">";
  return name.c_str();
}

// Workgroups of the instantiation that are resident on one compute unit
// (from its register use; cached per device, host threads storing the same
// value).
template <int NCHUNK, bool FULL, bool PER_HEAD>
int resident_groups_per_cu() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, qk_prologue_kernel<NCHUNK, FULL, PER_HEAD>,
                                                     kWavesPerBlock * 64, 0) !=
            hipSuccess ||
        n < 1)
      n = 1;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// One resident round of waves, at most one wave per row.
template <int NCHUNK, bool FULL, bool PER_HEAD>
int launch_rows(const PrologueArgs& a, hipStream_t st, const char** launched) {
  const int64_t rows = (int64_t)a.B * a.S;
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const int64_t groups = std::min<int64_t>((rows + kWavesPerBlock - 1) / kWavesPerBlock,
                                           cus * resident_groups_per_cu<NCHUNK, FULL, PER_HEAD>());
  hipLaunchKernelGGL((qk_prologue_kernel<NCHUNK, FULL, PER_HEAD>), dim3((unsigned)groups),
                     dim3(kWavesPerBlock * 64), 0, st, a);
  *launched = prologue_kernel_name<NCHUNK, FULL, PER_HEAD>();
  return (int)hipGetLastError();
}

template <int NCHUNK, bool PER_HEAD>
int launch_ph(const PrologueArgs& a, hipStream_t st, const char** launched) {
  return (a.H * a.D) % 512 == 0 ? launch_rows<NCHUNK, true, PER_HEAD>(a, st, launched)
                                : launch_rows<NCHUNK, false, PER_HEAD>(a, st, launched);
}

template <int NCHUNK>
int launch(const PrologueArgs& a, hipStream_t st, const char** launched) {
  // (without a weight the norm is skipped and PER_HEAD has no effect)
  return a.per_head && a.weight != nullptr ? launch_ph<NCHUNK, true>(a, st, launched)
                                           : launch_ph<NCHUNK, false>(a, st, launched);
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
