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
void na3d_wave_kernel(const Na3dArgs a, int n_yb, int n_xb, int n_xg) {
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
      const float mneg = -m_run;
#pragma unroll
      for (int r = 0; r < 8; ++r) pv[r] = (bf16)fast_exp2(S[8 * j + r] + mneg);
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


// ---------------------------------------------------------------------------
// Row-streaming kernel (kw' <= 25). A workgroup of 8 waves owns a brick of
// 1 (t) x 8 (y) x 32 (x) queries of one head: waves 0-3 take y rows 0-3 and
// waves 4-7 rows 4-7, each wave 8 consecutive x. The union of the brick's
// windows is kt' x NY key rows (t', y') of NX consecutive x positions. The
// workgroup streams those rows two at a time through LDS with the DMA path
// (NBUF-deep ring, issued NBUF-1 steps ahead); each wave reads the SEG-wide
// window of x positions it needs from every row: one 32-key chunk per step
// for SEG = 16 (two rows x 16), two chunks for SEG = 32 (one row each).
// Waves whose y window misses both rows of a step skip its math.

template <int SEG, int NBUF>
struct RowCfg {
  static constexpr int kWaves = 8;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kBrickY = 8, kBrickX = 32;
  static constexpr int kNS = SEG == 16 ? 40 : 64;             // key slots per LDS row
  static constexpr int kRowTensorBytes = kNS * kRowBytes;     // one key row of K (or V)
  static constexpr int kStepBytes = 4 * kRowTensorBytes;      // K row0, K row1, V row0, V row1
  static constexpr int kSmem = NBUF * kStepBytes;
  static constexpr int kDmaTotal = kNS;                        // 1 KiB DMA copies per step
  static constexpr int kDmaPerWave = (kDmaTotal + kWaves - 1) / kWaves;  // per wave (last ones repeat)
};

__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_row) {
  // Issued as inline assembly so the compiler does not wait for the copy
  // before every later LDS read; the kernel orders it with s_waitcnt and a
  // barrier before any wave reads the destination.
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_row))
               : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

template <int SEG, int NBUF>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void na3d_rows_kernel(const Na3dArgs a, int n_yb, int n_xb) {
  using C = RowCfg<SEG, NBUF>;
  constexpr int RT = C::kRowTensorBytes;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::kSmem];
  VX_LDS unsigned char* const lds = (VX_LDS unsigned char*)smem;
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int hf = lane >> 5;
  const int col = lane & 31;

  // Workgroups are dispatched round-robin over the 8 XCDs (each with its own
  // L2). With heads % 8 == 0 the linear workgroup id is remapped so that XCD
  // x walks the bricks of heads x, x+8, ... in order: the workgroups resident
  // on one XCD then cover neighbouring bricks of one head and share their
  // key rows in that XCD's L2.
  const int n_bricks = a.T * n_yb * n_xb;
  int brick, head;
  if ((a.NH & 7) == 0) {
    const int lin = blockIdx.y * n_bricks + blockIdx.x;  // launch order within a batch item
    const int xcd = lin & 7, j = lin >> 3;
    head = xcd + 8 * (j / n_bricks);
    brick = j % n_bricks;
  } else {
    head = blockIdx.y;
    brick = blockIdx.x;
  }
  const int xb = brick % n_xb;
  const int yb = (brick / n_xb) % n_yb;
  const int t = brick / (n_xb * n_yb);
  const int b = blockIdx.z;
  const int T = a.T, Hs = a.Hs, W = a.W, kt = a.kt, kh = a.kh, kw = a.kw;
  const int y0 = yb * C::kBrickY, x0 = xb * C::kBrickX;

  // ---- the workgroup's key rows.
  const int t_lo = window_start(t, T, kt);
  const int Y_lo = window_start(y0, Hs, kh);
  const int NY = window_start(min(y0 + C::kBrickY - 1, Hs - 1), Hs, kh) + kh - Y_lo;
  const int X_lo = window_start(x0, W, kw);
  const int nrows = kt * NY;
  const int n_steps = (nrows + 1) / 2;

  // ---- this wave's queries: y rows yq0..yq0+3, x columns xq0..xq0+7.
  const int yq0 = y0 + 4 * (wave >> 2);
  const int xq0 = x0 + 8 * (wave & 3);
  const bool wave_live = yq0 < Hs && xq0 < W;
  const int yw_lo = window_start(min(yq0, Hs - 1), Hs, kh) - Y_lo;          // wave's y window, in
  const int yw_hi = window_start(min(yq0 + 3, Hs - 1), Hs, kh) + kh - Y_lo;  // box rows
  const int ox = window_start(min(xq0, W - 1), W, kw) - X_lo;  // wave's first x slot

  // ---- this lane's query and its window.
  const int yq = yq0 + col / 8, xq = xq0 + col % 8;
  const bool q_in = yq < Hs && xq < W;
  const int yqc = min(yq, Hs - 1), xqc = min(xq, W - 1);
  const int sy = window_start(yqc, Hs, kh) - Y_lo;
  const int sx = window_start(xqc, W, kw) - X_lo - ox;  // in [0, SEG - kw]
  // Per score register i: +inf if its key's x slot lies in this lane's
  // window, -inf otherwise (the mask is a v_min3 with the row limit below).
  float xlim[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int p = (SEG == 16 ? ((i >> 2) & 1) * 8 : (i >> 2) * 8) + hf * 4 + (i & 3);
    xlim[i] = (unsigned)(p - sx) < (unsigned)kw ? __builtin_inff() : -__builtin_inff();
  }

  const int64_t tok_stride = (int64_t)a.NH * kD;
  const int64_t head_off = (int64_t)b * T * Hs * W * tok_stride + (int64_t)head * kD;
  const bf16* qg = (const bf16*)a.q + head_off;
  const bf16* kg = (const bf16*)a.k + head_off;
  const bf16* vg = (const bf16*)a.v + head_off;
  bf16* og = (bf16*)a.o + head_off;
  auto token = [&](int tt, int yy, int xx) -> int64_t { return ((int64_t)tt * Hs + yy) * W + xx; };

  bf16x8 qr[8];
  {
    const bf16* p = qg + token(t, yqc, xqc) * tok_stride + hf * 8;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) qr[ds] = *(const bf16x8*)(p + ds * 16);
  }

  // ---- DMA of step s into ring slot s % NBUF: copy i of the step covers
  // tensor i / (kNS/2), row i / (kNS/4) % 2 and x slots 4*(i % (kNS/4)) + 0..3.
  // The lane-dependent part of every copy's source address (x position and
  // swizzled 16-byte chunk) is fixed for the workgroup; only the row token
  // changes per step and is computed once per step in scalar registers.
  const int srow = lane >> 4, scol = lane & 15;
  int64_t dma_off[C::kDmaPerWave];
#pragma unroll
  for (int p = 0; p < C::kDmaPerWave; ++p) {
    // copies past kDmaTotal repeat the last one (same bytes, same place), so
    // every wave issues the same number of copies per step
    const int i = min(wave * C::kDmaPerWave + p, C::kDmaTotal - 1);
    const int pos = 4 * (i % (C::kNS / 4)) + srow;
    dma_off[p] = (int64_t)min(X_lo + pos, W - 1) * tok_stride + ((scol ^ row_swizzle(pos)) * 8);
  }
  // (t', y') of box row r as a token offset, and its y index within the box.
  auto row_token = [&](int r, int& yr) -> int64_t {
    const int tr = r / NY;
    yr = r - tr * NY;
    return (((int64_t)(t_lo + tr) * Hs + (Y_lo + yr)) * W) * tok_stride;
  };
  auto issue_step = [&](int s) {
    const int slot = s % NBUF;
    int yr_unused;
    const int64_t rt0 = row_token(min(2 * s, nrows - 1), yr_unused);
    const int64_t rt1 = row_token(min(2 * s + 1, nrows - 1), yr_unused);
#pragma unroll
    for (int p = 0; p < C::kDmaPerWave; ++p) {
      const int i = min(wave * C::kDmaPerWave + p, C::kDmaTotal - 1);
      const int tensor = i / (C::kNS / 2);
      const int rowsel = (i / (C::kNS / 4)) & 1;
      const int g = i % (C::kNS / 4);
      const bf16* src = (tensor ? vg : kg) + (rowsel ? rt1 : rt0) + dma_off[p];
      const int dst = slot * C::kStepBytes + (2 * tensor + rowsel) * RT + 4 * g * kRowBytes;
      lds_dma16(src, lds_base + dst);
    }
  };

  // ---- per-lane LDS offsets. K fragment: key col of the chunk.
  int kbase, ksw;
  if (SEG == 16) {
    const int pos = ox + (col & 15);
    kbase = (col >> 4) * RT + pos * kRowBytes;
    ksw = row_swizzle(pos);
  } else {
    const int pos = ox + col;
    kbase = pos * kRowBytes;
    ksw = row_swizzle(pos);
  }
  int koff[4];
#pragma unroll
  for (int d4 = 0; d4 < 4; ++d4) koff[d4] = kbase + (((2 * d4 + hf) ^ ksw) * 16);
  // V transpose reads: key 16j + 8e + 4hf + vr of the chunk.
  const int i16 = lane & 15;
  const int vr = i16 >> 2, vc = i16 & 3, dh = (lane >> 4) & 1;
  int voff[2][2];  // [e][db & 1]
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int pos = ox + 8 * e + 4 * hf + vr;
    const int sw = row_swizzle(pos);
#pragma unroll
    for (int db1 = 0; db1 < 2; ++db1)
      voff[e][db1] = 2 * RT + pos * kRowBytes + (((4 * db1 + 2 * dh + (vc >> 1)) ^ sw) * 16) + (vc & 1) * 8;
  }

  f32x16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;
  const float c2 = a.scale * kLog2e;

  // One 32-key chunk: K rows at kaddr + koff, V rows at vaddr + voff; rows
  // r0 (keys 0-15) and r1 (keys 16-31) of the box, x slots from this
  // wave's window (SEG = 16), or one row r0 for all 32 keys (SEG = 32).
  // ok0/ok1: the chunk's first / second 16 keys come from an existing box
  // row; yr0/yr1: those rows' y index within the box.
  auto chunk = [&](const VX_LDS unsigned char* kaddr, const VX_LDS unsigned char* vaddr, bool ok0, int yr0,
                   bool ok1, int yr1) {
    f32x16 S = f32x16{};
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
      const bf16x8 kf = *(const VX_LDS bf16x8*)(kaddr + koff[ds & 3] + (ds >> 2) * 128);
      S = mfma32x32x16(kf, qr[ds], S);
    }
    // window mask: keys outside this lane's y or x window -> -inf
    float rlim[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int yr = h2 == 0 ? yr0 : yr1;
      const bool row_ok = (h2 == 0 ? ok0 : ok1) && (unsigned)(yr - sy) < (unsigned)kh;
      rlim[h2] = row_ok ? __builtin_inff() : -__builtin_inff();
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) S[i] = __builtin_fminf(__builtin_fminf(S[i], xlim[i]), rlim[i >> 3]);
    float mx = S[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = __builtin_fmaxf(mx, S[i]);
    const float ms = halves_max(mx) * c2;  // scores stay raw; c2 folds into the exp argument
    if (__builtin_amdgcn_ballot_w64(ms > m_run + kRescaleSlack) != 0) {
      const float mn = __builtin_fmaxf(m_run, ms);
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
      const float mneg = -m_run;
#pragma unroll
      for (int r = 0; r < 8; ++r) pv[r] = (bf16)fast_exp2(__builtin_fmaf(S[8 * j + r], c2, mneg));
      P[j] = pv;
      l_run = sum8(pv, l_run);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int jo = SEG == 16 ? j * RT : j * 16 * kRowBytes;
        const VX_LDS unsigned char* p0 = vaddr + jo + voff[0][db & 1] + (db >> 1) * 128;
        const VX_LDS unsigned char* p1 = vaddr + jo + voff[1][db & 1] + (db >> 1) * 128;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)p0);
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)p1);
        const bf16x8 vf = concat(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi));
        O[db] = mfma32x32x16(vf, P[j], O[db]);
      }
  };

  // ---- prologue: the first NBUF-1 steps in flight.
#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s) issue_step(min(s, n_steps - 1));
  for (int s = 0; s < n_steps; ++s) {
    // Step s landed once only the NBUF-2 most recent steps may be in flight.
    wait_vmem<C::kDmaPerWave * (NBUF - 2)>();
    __syncthreads();
    // The slot of step s-1 is free now: refill it with step s+NBUF-1.
    issue_step(min(s + NBUF - 1, n_steps - 1));
    int y0r, y1r;
    (void)row_token(2 * s, y0r);
    (void)row_token(min(2 * s + 1, nrows - 1), y1r);
    const bool ok1 = 2 * s + 1 < nrows;
    const bool live = wave_live && ((y0r >= yw_lo && y0r < yw_hi) || (ok1 && y1r >= yw_lo && y1r < yw_hi));
    if (live) {
      const VX_LDS unsigned char* base = lds + (s % NBUF) * C::kStepBytes;
      if (SEG == 16) {
        chunk(base, base, true, y0r, ok1, y1r);
      } else {
        chunk(base, base, true, y0r, true, y0r);
        chunk(base + RT, base + RT, ok1, y1r, ok1, y1r);
      }
    }
  }
  wait_vmem<0>();

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
  hipStream_t st = (hipStream_t)stream;
  if (a.kw <= 25) {
    const int n_yb = (a.Hs + 7) / 8;
    const int n_xb = (a.W + 31) / 32;
    dim3 grid((unsigned)a.T * n_yb * n_xb, a.NH, a.B);
    if (a.kw <= 9)
      hipLaunchKernelGGL((na3d_rows_kernel<16, 4>), grid, dim3(512), 0, st, a, n_yb, n_xb);
    else
      hipLaunchKernelGGL((na3d_rows_kernel<32, 2>), grid, dim3(512), 0, st, a, n_yb, n_xb);
    return (int)hipGetLastError();
  }
  const int n_yb = (a.Hs + kBrickY - 1) / kBrickY;
  const int n_xb = (a.W + kBrickX - 1) / kBrickX;
  const int n_xg = (n_xb + kWaves - 1) / kWaves;
  dim3 grid((unsigned)a.T * n_yb * n_xg, a.NH, a.B);
  hipLaunchKernelGGL(na3d_wave_kernel, grid, dim3(kWaves * 64), 0, st, a, n_yb, n_xb, n_xg);
  return (int)hipGetLastError();
}

}  // namespace vx
