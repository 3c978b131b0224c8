// 3D neighbourhood attention forward for gfx950 (NATTEN semantics with
// boundary-clamped windows), bf16 in/out, D = 128.
//
// Each wave owns a query brick of 1 (t) x 4 (y) x 8 (x) = 32 queries of one
// head. Because the brick spans a single t, every query in it shares the t
// window, and the union of the bricks' windows is a (kt', ny, nx) box of
// keys with ny <= 3 + kh' and nx <= 7 + kw'. The wave walks that box in
// chunks of 32 keys, laid out as (t', y') rows of SEG = round_up(nx, 16)
// x-positions, so every 16-key half chunk lies inside one (t', y') row. Per
// chunk it computes S^T = K Q^T with bf16 MFMA (K fragments loaded straight
// from global memory), masks every (query, key) pair outside the query's own
// window to -inf, runs the same lazy-rescale online softmax as the flash
// kernel, and accumulates O^T += V^T P^T with V staged through a
// wave-private, double-buffered LDS slot and read back with the transpose
// read. Waves never synchronise with each other.
#include "vx_gfx950.hpp"
#include "vx_kernels.h"

namespace vx {
namespace {

constexpr int kD = 128;
constexpr int kRowBytes = kD * 2;
constexpr int kChunk = 32;                       // keys per chunk
constexpr int kChunkBytes = kChunk * kRowBytes;  // 8 KiB
constexpr int kBrickY = 4;
constexpr int kBrickX = 8;
constexpr int kWaves = 4;
constexpr float kRescaleSlack = 8.0f;
constexpr float kNegBig = -1.0e30f;

__device__ __forceinline__ int row_swizzle(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

__device__ __forceinline__ int window_start(int i, int len, int k) {
  return min(max(i - k / 2, 0), len - k);
}

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 2)))
void na3d_fwd_kernel(const Na3dArgs a, int n_yb, int n_xb, int n_xg) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kWaves * 2 * kChunkBytes];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hf = lane >> 5;
  const int col = lane & 31;

  // ---- which brick: blockIdx.x = (t * n_yb + yb) * n_xg + xg, wave -> xb.
  int bid = blockIdx.x;
  const int xg = bid % n_xg;
  bid /= n_xg;
  const int yb = bid % n_yb;
  const int t = bid / n_yb;
  const int xb = xg * kWaves + wave;
  if (xb >= n_xb) return;  // whole wave; no workgroup barrier is used below
  const int head = blockIdx.y;
  const int b = blockIdx.z;
  const int T = a.T, Hs = a.Hs, W = a.W, kt = a.kt, kh = a.kh, kw = a.kw;
  const int y0 = yb * kBrickY, x0 = xb * kBrickX;

  // ---- the brick's key box.
  const int t_lo = window_start(t, T, kt);
  const int y_lo = window_start(y0, Hs, kh);
  const int ny = window_start(min(y0 + kBrickY - 1, Hs - 1), Hs, kh) + kh - y_lo;
  const int x_lo = window_start(x0, W, kw);
  const int nx = window_start(min(x0 + kBrickX - 1, W - 1), W, kw) + kw - x_lo;
  const int seg = (nx + 15) & ~15;  // <= 64 (checked on the host)
  const int nrows = kt * ny;
  const int n_chunks = (nrows * seg + kChunk - 1) / kChunk;

  // ---- this lane's query and its window relative to the box.
  const int yq = y0 + col / kBrickX, xq = x0 + col % kBrickX;
  const bool q_in = yq < Hs && xq < W;
  const int yqc = min(yq, Hs - 1), xqc = min(xq, W - 1);
  const int sy = window_start(yqc, Hs, kh) - y_lo;
  const int sx = window_start(xqc, W, kw) - x_lo;
  const uint64_t xmask = (kw >= 64 ? ~0ull : ((1ull << kw) - 1)) << sx;

  const int64_t tok_stride = (int64_t)a.NH * kD;  // elements between tokens
  const int64_t plane = (int64_t)T * Hs * W;
  const int64_t head_off = (int64_t)b * plane * tok_stride + (int64_t)head * kD;
  const bf16* qg = (const bf16*)a.q + head_off;
  const bf16* kg = (const bf16*)a.k + head_off;
  const bf16* vg = (const bf16*)a.v + head_off;
  bf16* og = (bf16*)a.o + head_off;
  auto token = [&](int tt, int yy, int xx) -> int64_t { return ((int64_t)tt * Hs + yy) * W + xx; };

  // ---- Q fragments (B operand), resident.
  bf16x8 qr[8];
  {
    const bf16* p = qg + token(t, yqc, xqc) * tok_stride + hf * 8;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) qr[ds] = *(const bf16x8*)(p + ds * 16);
  }

  // Token index of key j of a 16-key half chunk starting at box key kb2.
  auto half_row = [&](int kb2, int& trow, int& j0) {
    int row = kb2 / seg;
    j0 = kb2 - row * seg;
    row = min(row, nrows - 1);
    trow = row;
  };
  auto row_token = [&](int row, int j) -> int64_t {
    const int tr = row / ny, yr = row - tr * ny;
    return token(t_lo + tr, y_lo + yr, min(x_lo + j, W - 1));
  };

  // K fragment of chunk c for this lane: key row col of the chunk.
  bf16x8 kf[8], kfn[8];
  auto load_k = [&](int c, bf16x8* dst) {
    int row, j0;
    half_row(c * kChunk + (col & 16), row, j0);
    const bf16* p = kg + row_token(row, j0 + (col & 15)) * tok_stride + hf * 8;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) dst[ds] = *(const bf16x8*)(p + ds * 16);
  };
  // V rows of chunk c: lane covers rows 4p + lane/16 (p = 0..7), 16-byte column lane%16.
  u32x4 vst[8];
  auto load_v = [&](int c) {
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      int row, j0;
      half_row(c * kChunk + 16 * h2, row, j0);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int r = 4 * p + (lane >> 4);  // row within the half chunk
        const bf16* src = vg + row_token(row, j0 + r) * tok_stride + (lane & 15) * 8;
        vst[4 * h2 + p] = *(const u32x4*)src;
      }
    }
  };
  unsigned char* const vbuf0 = smem + wave * 2 * kChunkBytes;
  unsigned char* const vbuf1 = vbuf0 + kChunkBytes;
  auto store_v = [&](unsigned char* buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 16 * (i >> 2) + 4 * (i & 3) + (lane >> 4);
      *(u32x4*)(buf + r * kRowBytes + (((lane & 15) ^ row_swizzle(r)) * 16)) = vst[i];
    }
  };
  // V transpose-read offsets (same layout as the flash kernel).
  const int i16 = lane & 15;
  const int vr = i16 >> 2, vc = i16 & 3, dh = (lane >> 4) & 1;
  const int vsw = 2 * vr + hf;
  int voff[2];
#pragma unroll
  for (int db1 = 0; db1 < 2; ++db1)
    voff[db1] = (hf * 4 + vr) * kRowBytes + (((4 * db1 + 2 * dh + (vc >> 1)) ^ vsw) * 16) + (vc & 1) * 8;

  f32x16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;
  const float c2 = a.scale * kLog2e;

  load_k(0, kf);
  load_v(0);
  store_v(vbuf0);
  for (int c = 0; c < n_chunks; ++c) {
    const bool has_next = c + 1 < n_chunks;
    if (has_next) {
      load_k(c + 1, kfn);
      load_v(c + 1);
    }
    f32x16 S = f32x16{};
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) S = mfma32x32x16(kf[ds], qr[ds], S);

    // ---- window mask, scores to log2 units.
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int kb2 = c * kChunk + 16 * h2;
      const int row = kb2 / seg;
      const int j0 = kb2 - row * seg;
      const int tr = row / ny, yr = row - tr * ny;
      const bool row_ok = row < nrows && (unsigned)(yr - sy) < (unsigned)kh;
      (void)tr;  // every key row of the box is inside the brick's t window
      const uint64_t xm = row_ok ? (xmask >> (j0 + hf * 4)) : 0ull;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int bit = (i >> 2) * 8 + (i & 3);
        const bool ok = (xm >> bit) & 1ull;
        const float sv = S[8 * h2 + i] * c2;
        S[8 * h2 + i] = ok ? sv : -__builtin_inff();
      }
    }

    // ---- online softmax (lazy rescale).
    float mx = S[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, S[i]);
    const float ms = halves_max(mx);
    if (__builtin_amdgcn_ballot_w64(ms > m_run + kRescaleSlack) != 0) {
      const float mn = fmaxf(m_run, ms);
      const float alpha = fast_exp2(m_run - mn);
      m_run = mn;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) O[db] *= alpha;
    }
    bf16x8 P[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8 pv;
#pragma unroll
      for (int r = 0; r < 8; ++r) pv[r] = (bf16)fast_exp2(S[8 * j + r] - m_run);
      P[j] = pv;
      l_run = sum8(pv, l_run);
    }

    // ---- O^T += V^T P^T.
    const unsigned char* vb = (c & 1) ? vbuf1 : vbuf0;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const unsigned char* base = vb + (16 * j) * kRowBytes + (db >> 1) * 128 + voff[db & 1];
        const bf16x8 vf = concat(lds_read_tr16(base), lds_read_tr16(base + 8 * kRowBytes));
        O[db] = mfma32x32x16(vf, P[j], O[db]);
      }

    if (has_next) {
      store_v((c & 1) ? vbuf0 : vbuf1);
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) kf[ds] = kfn[ds];
    }
  }

  const float lt = halves_sum(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (q_in) {
    bf16* orow = og + token(t, yq, xq) * tok_stride;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (bf16)(O[db][g * 4 + e] * inv);
        *(bf16x4*)(orow + db * 32 + g * 8 + hf * 4) = ov;
      }
  }
}

}  // namespace

int launch_na3d_fwd(const Na3dArgs& a, void* stream) {
  if (a.D != kD) return (int)hipErrorNotSupported;
  const int n_yb = (a.Hs + kBrickY - 1) / kBrickY;
  const int n_xb = (a.W + kBrickX - 1) / kBrickX;
  const int n_xg = (n_xb + kWaves - 1) / kWaves;
  dim3 grid((unsigned)a.T * n_yb * n_xg, a.NH, a.B);
  hipLaunchKernelGGL(na3d_fwd_kernel, grid, dim3(kWaves * 64), 0, (hipStream_t)stream, a, n_yb, n_xb, n_xg);
  return (int)hipGetLastError();
}

}  // namespace vx
