// 3D neighbourhood attention forward for gfx950 (NATTEN semantics with
// boundary-clamped windows), bf16 in/out, head dim 128 or 64.
//
// Three kernels, chosen by the clamped x window kw' (the launch plan of the
// C ABI, Na3dVariant; at head dim 64 also by how the grid's y x x plane
// rounds up to each brick shape):
// - na3d_pipe_kernel<SEG, D> (kw' <= 9 or 13 < kw' <= 25): a workgroup of 4
//   waves owns a 1 (t) x 4 (y) x 32 (x) query brick of one head and streams
//   the union of its windows, kt' x NY key rows (t', y'), through LDS with
//   the DMA copy path; each wave reads the SEG-wide x window its 4 x 8
//   queries need, 32 keys per step, and runs the flash kernel's software
//   pipeline (QK^T of the next chunk and PV of the previous one interleaved
//   with the masking and lazy-rescale softmax of the current one).
//   na3d_tstack_kernel<128> (kw' <= 9 with t windows of 2 and more, head dim
//   128) runs the same body on 2 x 4 x 16 bricks, two 4 x 8 waves per t
//   plane sharing one stream of kt' + 1 planes of 24-key rows (30 % fewer
//   copied rows per query at a (3,7,7) window, no half-empty brick at
//   widths of a multiple of 16); a wave whose t window misses the chunks
//   around a step only copies.
// - na3d_tall_kernel<D> (9 < kw' <= 13, and kw' <= 9 at head dim 64 when
//   its bricks pad the grid no more): the same body on 1 x 8 x 16 bricks
//   with waves of 8 y x 4 x queries, so that a wave's x window still fits a
//   16-key segment; na3d_tall_wide_kernel<64> runs 1 x 8 x 32 bricks of 8
//   such waves at head dim 64, and na3d_deep_kernel<64> (t windows of 5
//   and more) 2 x 4 x 32 bricks of waves of 2 t x 4 y x 4 x queries.
// - na3d_wave_kernel<D> (kw' > 25, any size, D 128 or 64): each wave owns a
//   1 x 4 x 8 brick on its own and walks its (kt', ny, nx) key box in chunks
//   of 32 keys, laid out as (t', y') rows of SEG = round_up(nx, 16)
//   x-positions, with K fragments loaded straight from global memory and V
//   staged through a wave-private, double-buffered LDS slot; its waves never
//   synchronise with each other.
// In all three, every (query, key) pair outside the query's own window is
// set to -inf before the exponent, so each query attends exactly its
// kt' x kh' x kw' window.
#include "vx_gfx950.hpp"
#include "vx_kernels.h"
#include "vx_qk_prep.hpp"

namespace vx {
namespace {

constexpr int kChunk = 32;  // keys per chunk of the per-wave kernel
constexpr int kBrickY = 4;
constexpr int kBrickX = 8;
constexpr int kWaves = 4;
constexpr float kRescaleSlack = 8.0f;
constexpr float kSumLimit = 256.0f;  // 2^kRescaleSlack
constexpr float kNegBig = -1.0e30f;

__device__ __forceinline__ int row_swizzle(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }


__device__ __forceinline__ int window_start(int i, int len, int k) {
  return min(max(i - k / 2, 0), len - k);
}

// Sum of a lane's 16 fp32 probabilities (pairwise).
__device__ __forceinline__ float sum16(const float (&p)[16]) {
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = p[2 * i] + p[2 * i + 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = q[2 * i] + q[2 * i + 1];
  return (q[0] + q[1]) + (q[2] + q[3]);
}

// The block's q preparation on the resident Q fragments of one lane (query
// `tok`, d = 16 * ds + 8 * hf + 0..7 in qr[ds]; lane l ^ 32 holds the other
// half of the row), with the rounding points of the one-pass prologue kernel.
// The per-head sum of squares adds the 8-element chunk sums in the order of
// that kernel's xor-butterfly over the head's D/8 chunks (chunk c = 2*ds+hf
// pairs with c^8, c^4, c^2 inside the lane and with c^1 in the other half).
// Output rows of a wave's 32 queries, query r being the token (t + r /
// (QX QY), y0 + r / QX % QY, x0 + r % QX) of the head's output og (tokens
// tok_stride apart; rows outside the T x Hs x W grid are dropped): the O^T
// accumulators normalised by inv, packed and regrouped into whole 128-byte
// lines (pack_out_rows, line_chunks), one 64-wide d pair at a time.
template <int kDB, int QX, int QY = 32 / QX>
__device__ __forceinline__ void store_na_rows(const f32x16 (&O)[kDB], float inv, bf16* og, int64_t tok_stride,
                                              int t, int y0, int x0, int T, int Hs, int W, int lane) {
#pragma unroll
  for (int p = 0; p < kDB / 2; ++p) {
    u32x4 c2[2][2];
    const f32x16 Ob[2] = {O[2 * p], O[2 * p + 1]};
    pack_out_rows<2>(Ob, inv, c2);  // all lanes: cross-lane exchanges
    u32x4 out[4];
    line_chunks(c2, out);
    const uint32_t cofs = line_chunk_offset(lane, p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (lane & 7) + 8 * i;
      const int tt = t + r / (QX * QY), y = y0 + r / QX % QY, x = x0 + r % QX;
      if (tt < T && y < Hs && x < W)
        *(u32x4*)((unsigned char*)(og + (((int64_t)tt * Hs + y) * W + x) * tok_stride) + cofs) = out[i];
    }
  }
}

template <int NDS>
__device__ __forceinline__ void prep_q(bf16x8 (&qr)[NDS], int hf, int64_t tok, int tq, int yq, int xq,
                                       const Na3dArgs& a) {
  constexpr int D = NDS * 16;
  // all loads first (weights, then the token's rotation tables), so their
  // latencies overlap
  f32x4 w[NDS][2], cs[NDS], sn[NDS];
  const bool norm = (a.q_prep & kQPrepNorm) != 0, rope = (a.q_prep & kQPrepRope) != 0;
  if (norm) {
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const float* wp = a.q_weight + ds * 16 + hf * 8;
      w[ds][0] = *(const f32x4*)wp;
      w[ds][1] = *(const f32x4*)(wp + 4);
    }
  }
  if (rope && (a.q_prep & kQPrepRopeAxes)) {
    // per-axis rows (t rows, then h rows, then w rows of one table): the
    // lane's 4 pairs 8 ds + 4 hf + 0..3 lie in one axis's part (its
    // boundaries are multiples of 4) and are read at their own columns of
    // that axis's row; a few hundred rows shared by every token and head
    // instead of one table row per token. 32-bit element offsets.
    const int st = (int)a.q_tab_stride;
    const int row_t = tq * st, row_h = (a.T + yq) * st, row_w = (a.T + a.Hs + xq) * st;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int j = ds * 8 + hf * 4;
      const int off = (j < a.q_ax_pairs[0] ? row_t : (j < a.q_ax_pairs[1] ? row_h : row_w)) + j;
      cs[ds] = *(const f32x4*)(a.q_cos + off);
      sn[ds] = *(const f32x4*)(a.q_sin + off);
    }
  } else if (rope) {
    const float* cr = a.q_cos + tok * a.q_tab_stride + hf * 4;
    const float* sr = a.q_sin + tok * a.q_tab_stride + hf * 4;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      cs[ds] = *(const f32x4*)(cr + ds * 8);
      sn[ds] = *(const f32x4*)(sr + ds * 8);
    }
  }
  if (norm) {
    float ss[NDS];
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) ss[ds] = sum_sq8(qr[ds]);
    // level m adds ds and ds + m (m = NDS/2, ..., 1); ss[0] ends with the sum
#pragma unroll
    for (int m = NDS / 2; m >= 1; m >>= 1)
#pragma unroll
      for (int ds = 0; ds < m; ++ds) ss[ds] = ss[ds] + ss[ds + m];
    const float rinv = rms_inv(halves_sum(ss[0]), D, a.q_eps);
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
      for (int e = 0; e < 8; ++e) qr[ds][e] = rms_elem((float)qr[ds][e], rinv, w[ds][e >> 2][e & 3]);
  }
  if (a.q_prep & kQPrepScale) {
    const float ps = (float)(bf16)a.q_post_scale;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
      for (int e = 0; e < 8; ++e) qr[ds][e] = scale_elem((float)qr[ds][e], ps);
  }
  if (rope) {
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
      for (int p = 0; p < 4; ++p) rope_pair(qr[ds], p, cs[ds][p], sn[ds][p]);
  }
}

// Two waves per SIMD (at most 256 registers a wave; 230 at D = 128, no
// spills): its waves stream K from global memory, so the second wave covers
// those loads' latency (at D = 128 the kernel had 346 registers and one wave
// per SIMD: 1.9x slower at a (3,7,31) window).
template <int D>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void na3d_wave_kernel(const Na3dArgs a, int n_yb, int n_xb, int n_xg) {
  constexpr int kRB = D * 2;              // bytes of one key
  constexpr int kCB = kChunk * kRB;       // one chunk of V in LDS
  constexpr int kNDS = D / 16, kNDB = D / 32;
  constexpr int kCPR = D / 8;             // 16-byte columns of a key row
  constexpr int kRPP = 64 / kCPR;         // V rows a wave stages per pass
  constexpr int kVPass = kChunk / kRPP;   // passes per chunk
  __shared__ __attribute__((aligned(16))) unsigned char smem[kWaves * 2 * kCB];
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

  // ---- the brick's key box: kt' x ny rows of seg = round_up(nx, 16) x slots.
  const int t_lo = window_start(t, T, kt);
  const int y_lo = window_start(y0, Hs, kh);
  const int ny = window_start(min(y0 + kBrickY - 1, Hs - 1), Hs, kh) + kh - y_lo;
  const int x_lo = window_start(x0, W, kw);
  const int nx = window_start(min(x0 + kBrickX - 1, W - 1), W, kw) + kw - x_lo;
  const int seg = (nx + 15) & ~15;
  const int nrows = kt * ny;
  const int n_chunks = (nrows * seg + kChunk - 1) / kChunk;

  // ---- this lane's query and its window relative to the box.
  const int yq = y0 + col / kBrickX, xq = x0 + col % kBrickX;
  const bool q_in = yq < Hs && xq < W;
  const int yqc = min(yq, Hs - 1), xqc = min(xq, W - 1);
  const int sy = window_start(yqc, Hs, kh) - y_lo;
  const int sx = window_start(xqc, W, kw) - x_lo;

  const int64_t tok_stride = (int64_t)a.NH * D;  // elements between tokens
  const int64_t plane = (int64_t)T * Hs * W;
  const int64_t head_off = (int64_t)b * plane * tok_stride + (int64_t)head * D;
  const bf16* qg = (const bf16*)a.q + head_off;
  const bf16* kg = (const bf16*)a.k + head_off;
  const bf16* vg = (const bf16*)a.v + head_off;
  bf16* og = (bf16*)a.o + head_off;
  auto token = [&](int tt, int yy, int xx) -> int64_t { return ((int64_t)tt * Hs + yy) * W + xx; };

  // ---- Q fragments (B operand), resident.
  bf16x8 qr[kNDS];
  {
    const bf16* p = qg + token(t, yqc, xqc) * tok_stride + hf * 8;
#pragma unroll
    for (int ds = 0; ds < kNDS; ++ds) qr[ds] = *(const bf16x8*)(p + ds * 16);
  }
  if (a.q_prep != 0) prep_q(qr, hf, token(t, yqc, xqc), t, yqc, xqc, a);

  // Box row and first x slot of the 16-key half chunk starting at box key kb2.
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

  // K fragment of chunk c for this lane: key row col of the chunk (one
  // register set: the next chunk's loads are issued once this chunk's QK^T
  // has read it).
  bf16x8 kf[kNDS];
  auto load_k = [&](int c, bf16x8* dst) {
    int row, j0;
    half_row(c * kChunk + (col & 16), row, j0);
    const bf16* p = kg + row_token(row, j0 + (col & 15)) * tok_stride + hf * 8;
#pragma unroll
    for (int ds = 0; ds < kNDS; ++ds) dst[ds] = *(const bf16x8*)(p + ds * 16);
  };
  // V rows of chunk c: pass p covers rows kRPP * p + lane / kCPR, 16-byte
  // column lane % kCPR (rows 0-15 from one box row, 16-31 from the next
  // half chunk's).
  u32x4 vst[kVPass];
  auto load_v = [&](int c) {
    int rowa, j0a, rowb, j0b;
    half_row(c * kChunk, rowa, j0a);
    half_row(c * kChunk + 16, rowb, j0b);
#pragma unroll
    for (int p = 0; p < kVPass; ++p) {
      const int r = kRPP * p + lane / kCPR;
      const bool second = r >= 16;
      const bf16* src = vg + row_token(second ? rowb : rowa, (second ? j0b : j0a) + (r & 15)) * tok_stride +
                        (lane % kCPR) * 8;
      vst[p] = *(const u32x4*)src;
    }
  };
  unsigned char* const vbuf0 = smem + wave * 2 * kCB;
  unsigned char* const vbuf1 = vbuf0 + kCB;
  auto store_v = [&](unsigned char* buf) {
#pragma unroll
    for (int p = 0; p < kVPass; ++p) {
      const int r = kRPP * p + lane / kCPR;
      *(u32x4*)(buf + r * kRB + (((lane % kCPR) ^ row_swizzle(r)) * 16)) = vst[p];
    }
  };
  // V transpose-read offsets (same layout as the flash kernel).
  const int i16 = lane & 15;
  const int vr = i16 >> 2, vc = i16 & 3, dh = (lane >> 4) & 1;
  const int vsw = 2 * vr + hf;
  int voff[2];
#pragma unroll
  for (int db1 = 0; db1 < 2; ++db1)
    voff[db1] = (hf * 4 + vr) * kRB + (((4 * db1 + 2 * dh + (vc >> 1)) ^ vsw) * 16) + (vc & 1) * 8;

  f32x16 O[kNDB];
#pragma unroll
  for (int db = 0; db < kNDB; ++db) O[db] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;
  const float c2 = a.scale * kLog2e;

  load_k(0, kf);
  load_v(0);
  store_v(vbuf0);
  for (int c = 0; c < n_chunks; ++c) {
    const bool has_next = c + 1 < n_chunks;
    if (has_next) load_v(c + 1);
    f32x16 S = f32x16{};
#pragma unroll
    for (int ds = 0; ds < kNDS; ++ds) S = mfma32x32x16(kf[ds], qr[ds], S);
    if (has_next) load_k(c + 1, kf);

    // ---- window mask, scores to log2 units. Score register i of half h2
    // holds x slot j0 + hf*4 + (i/4)*8 + i%4 of its box row.
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int kb2 = c * kChunk + 16 * h2;
      const int row = kb2 / seg;
      const int j0 = kb2 - row * seg;
      const int yr = row - (row / ny) * ny;
      const bool row_ok = row < nrows && (unsigned)(yr - sy) < (unsigned)kh;
      // (every key row of the box is inside the brick's t window)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int jx = j0 + hf * 4 + (i >> 2) * 8 + (i & 3);
        const bool ok = row_ok && (unsigned)(jx - sx) < (unsigned)kw;
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
      for (int db = 0; db < kNDB; ++db) O[db] *= alpha;
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
      for (int db = 0; db < kNDB; ++db) {
        const unsigned char* base = vb + (16 * j) * kRB + (db >> 1) * 128 + voff[db & 1];
        const bf16x8 vf = concat(lds_read_tr16(base), lds_read_tr16(base + 8 * kRB));
        O[db] = mfma32x32x16(vf, P[j], O[db]);
      }

    if (has_next) store_v((c & 1) ? vbuf0 : vbuf1);
  }

  const float lt = halves_sum(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  // (per-lane row stores: the line regrouping's registers would add spills
  // to this kernel at head dim 128)
  u32x4 chunk[kNDB][2];
  pack_out_rows<kNDB>(O, inv, chunk);  // all lanes: cross-lane exchange
  if (q_in) {
    bf16* orow = og + token(t, yq, xq) * tok_stride;
#pragma unroll
    for (int db = 0; db < kNDB; ++db)
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) *(u32x4*)(orow + db * 32 + (2 * pr + hf) * 8) = chunk[db][pr];
  }
}


// ---------------------------------------------------------------------------
// Pipelined row-streaming kernel (kw' <= 25). A workgroup of 4 waves owns a
// brick of 1 (t) x 4 (y) x 32 (x) queries of one head; wave w takes the 4 y
// rows and x columns 8w..8w+7. The union of the brick's windows is kt' x NY
// key rows (t', y') of at most 31 + kw' consecutive x positions, and every
// wave needs every row, so all waves run the same step sequence. The rows are
// streamed through LDS kRows at a time (2 rows for SEG = 16, 1 for SEG = 32),
// K and V in separate two-slot rings filled by the DMA path one step ahead;
// each wave reads the SEG-wide x window it needs from the step's rows, one
// 32-key chunk. Step s issues QK^T(s+1) and PV(s-1) as one block of
// D/16 + D/16 MFMA slots interleaved with the masking and softmax of chunk s
// (as in the flash kernel), so the matrix cores and the VALU work of a wave
// overlap. With at most 80 KiB of LDS and 256 VGPRs two workgroups share a
// CU. Head dims 128 and 64 (the LTX-2.5 diffusion VAE's) are instantiated.
//
// The tall geometry (TALL, SEG = 16, 9 < kw' <= 13) uses bricks of
// 1 x 8 (y) x 16 (x) with waves of 8 y rows x 4 x columns: a wave's x union
// (3 + kw' keys) still fits one 16-key segment, so a (11, 11, 11) window is
// scored with 18 rows x 16 keys per plane instead of the 14 x 32 of the
// 32-key segments.

// WIDE: tall bricks 32 x columns wide with 8 waves (each still 8 y x 4 x):
// the 42-key x union of a row is staged in 48 slots for 32 queries (26 in
// 32 for 16 with the narrow brick), one workgroup barrier per step for
// twice the queries.
// DEEP: wide bricks two t planes deep, 2 (t) x 4 (y) x 32 (x), waves of 2 t x
// 4 y x 4 x queries: for a t window of kt' planes the union of a wave's
// windows is (kt' + 1) x (kh' + 3) rows instead of kt' x (kh' + 7), e.g. 12 x
// 14 against 11 x 18 rows at (11, 11, 11).
// TSTACK: 2 (t) x 4 (y) x 16 (x) bricks whose four 4 y x 8 x waves sit two
// per t plane: one stream of (kt' + 1) planes serves both planes' waves, each
// scoring only the chunks of its own kt' planes (a wave none of whose rows
// in the previous, current and next chunk lies in its t window only copies).
template <int SEG, int D, bool TALL = false, bool WIDE = false, bool DEEP = false, bool TSTACK = false>
struct PipeCfg {
  static_assert(!TALL || SEG == 16, "the tall geometry reads 16-key segments");
  static_assert(!WIDE || TALL, "wide bricks are tall bricks");
  static_assert(!DEEP || WIDE, "deep bricks are wide bricks");
  static_assert(!TSTACK || (!TALL && SEG == 16), "t-stacked bricks hold 1 x 4 x 8 waves on 16-key segments");
  static constexpr bool kTStack = TSTACK;
  static constexpr int kWaves = WIDE ? 8 : 4;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kQT = DEEP || TSTACK ? 2 : 1;     // t planes per brick
  static constexpr int kWT = DEEP ? 2 : 1;               // t planes per wave
  static constexpr int kWX = TSTACK ? kWaves / 2 : kWaves;  // waves side by side in x
  static constexpr int kBrickY = TALL ? (DEEP ? 4 : 8) : 4;
  static constexpr int kBrickX = TALL ? (WIDE ? 32 : 16) : (TSTACK ? 16 : 32);
  static constexpr int kQX = kBrickX / kWX;              // x columns per wave
  static constexpr int kQY = 32 / (kQX * kWT);           // y rows per wave (and per brick)
  static constexpr int kRB = D * 2;                      // bytes of one key
  static constexpr int kRows = SEG == 16 ? 2 : 1;        // key rows per step
  // key slots per LDS row (>= kBrickX - kQX + SEG, a multiple of 8)
  static constexpr int kNS = TALL ? (WIDE ? 48 : 32) : (TSTACK ? 24 : (SEG == 16 ? 40 : 64));
  // An LDS key row is D/64 half-planes of kNS slots x 128 bytes (d 0-63,
  // then d 64-127); one 1 KiB DMA copy fills 8 slots of one half-plane.
  static constexpr int kHalfL = kNS * 128;               // one half-plane of a row
  static constexpr int kRowL = kNS * kRB;                // one LDS key row
  static constexpr int kKeysPerCopy = 8;
  static constexpr int kSlot = kRows * kRowL;            // one ring slot: one tensor, one step
  static constexpr int kK = 0, kV = 2 * kSlot;           // K slots 0,1 then V slots 0,1
  static constexpr int kSmem = 4 * kSlot;
  static constexpr int kCopies = kRows * kRowL / 1024;   // DMA copies per tensor per step
  // the copies of a step spread over the waves (those past kCopies are skipped;
  // every wait for them is a wait for all of a wave's copies)
  static constexpr int kCopiesPerWave = (kCopies + kWaves - 1) / kWaves;
  static constexpr int kQK = D / 16;                     // MFMAs of QK^T per chunk
  static constexpr int kPV = 2 * (D / 32);               // MFMAs of PV per chunk
  static constexpr int kSlots = kQK + kPV;
  static constexpr int kScoresPerSlot = 16 / kSlots;     // softmax work per slot (1 or 2)
  static_assert(kNS % kKeysPerCopy == 0 && kHalfL % 256 == 0, "whole copies per row, bank-aligned planes");
};

template <int SEG, int D, bool TALL, bool WIDE = false, bool DEEP = false, bool TSTACK = false>
__device__ __forceinline__ void na3d_pipe_body(const Na3dArgs& a, int n_yb, int n_xb) {
  using C = PipeCfg<SEG, D, TALL, WIDE, DEEP, TSTACK>;
  static_assert(C::kQY == C::kBrickY, "the waves of a t plane sit side by side in x");
  static_assert(C::kBrickX - C::kQX + SEG <= C::kNS, "a wave's segment stays inside the LDS row");
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
  const int n_tb = (a.T + C::kQT - 1) / C::kQT;  // t bricks
  const int n_bricks = n_tb * n_yb * n_xb;
  int brick, head;
  if (a.order == kNaOrderTColumns) {
    // Deep t windows: XCD x takes the x-th eighth of the (head, brick
    // column (y, x), t) sequence, t fastest, so its resident workgroups hold
    // bricks of consecutive t planes of one column, which share kt' - 1 of
    // their kt' key planes in that XCD's L2.
    const int total = n_bricks * a.NH;
    const int lin = blockIdx.y * n_bricks + blockIdx.x;  // launch order within a batch item
    const int xcd = lin & 7, j = lin >> 3;
    const int g = xcd * (total >> 3) + min(xcd, total & 7) + j;  // the eighths are contiguous ranges of g
    const int ncol = n_yb * n_xb;
    const int rest = g / n_tb;
    head = rest / ncol;
    brick = (g - rest * n_tb) * ncol + (rest - head * ncol);    // (tb * n_yb + yb) * n_xb + xb
  } else if ((a.NH & 7) == 0) {
    const int lin = blockIdx.y * n_bricks + blockIdx.x;  // launch order within a batch item
    const int xcd = lin & 7, j = lin >> 3;
    head = xcd + 8 * (j / n_bricks);
    brick = j % n_bricks;
  } else {
    head = blockIdx.y;
    brick = blockIdx.x;
  }
  // The integer divisions below run on the vector unit; their (uniform)
  // results go back to scalar registers, so the row walk stays scalar.
  auto uni = [](int x) { return __builtin_amdgcn_readfirstlane(x); };
  head = uni(head);
  const int xb = uni(brick % n_xb);
  const int yb = uni((brick / n_xb) % n_yb);
  const int t = uni(brick / (n_xb * n_yb)) * C::kQT;  // the brick's first t plane
  const int b = blockIdx.z;
  const int T = a.T, Hs = a.Hs, W = a.W, kt = a.kt, kh = a.kh, kw = a.kw;
  const int y0 = yb * C::kBrickY, x0 = xb * C::kBrickX;

  // ---- the workgroup's key rows (box rows r = tr * NY + yr over NT planes).
  const int t_lo = uni(window_start(t, T, kt));
  const int NT = C::kQT == 1 ? kt : uni(window_start(min(t + C::kQT - 1, T - 1), T, kt) + kt - t_lo);
  const int Y_lo = uni(window_start(y0, Hs, kh));
  const int NY = uni(window_start(min(y0 + C::kBrickY - 1, Hs - 1), Hs, kh) + kh - Y_lo);
  const int X_lo = uni(window_start(x0, W, kw));
  const int nrows = NT * NY;
  const int n_steps = (nrows + C::kRows - 1) / C::kRows;

  // ---- this wave's queries: t planes tw..tw+kWT-1 (tw = t, or t + 1 for the
  // second pair of t-stacked waves), y rows y0..y0+kBrickY-1, x columns
  // xq0..xq0+kQX-1.
  const int tw = t + wave / C::kWX;
  const int xq0 = x0 + C::kQX * (wave % C::kWX);
  const int ox = uni(window_start(min(xq0, W - 1), W, kw) - X_lo);  // wave's first x slot, <= kBrickX - kQX

  // ---- this lane's query and its window.
  const int tq = tw + col / (C::kQX * C::kQY), yq = y0 + col / C::kQX % C::kQY, xq = xq0 + col % C::kQX;
  const bool wave_in = y0 < Hs && xq0 < W && tw < T;  // wave-uniform: some query of the wave is in the grid
  const int tqc = min(tq, T - 1), yqc = min(yq, Hs - 1), xqc = min(xq, W - 1);
  const int sy = window_start(yqc, Hs, kh) - Y_lo;
  const int st = window_start(tqc, T, kt) - t_lo;  // (deep bricks: the lane's first plane in the box)
  const int sx = window_start(xqc, W, kw) - X_lo - ox;  // in [0, SEG - kw]
  // The x window of score register i (key (i/4)*8 + hf*4 + i%4 of the
  // chunk). kAccMask: a 0 / -inf vector that every chunk's QK^T MFMAs start
  // from (the first one's accumulator input), so the x window costs no
  // instruction per score. Otherwise (the tall bricks at head dim 64, whose
  // short steps need four waves per SIMD, i.e. at most 128 VGPRs, which the
  // extra accumulator input does not leave) a 0 / 0xffff mask per bf16 half
  // of each packed probability pair, one v_and_b32 per two scores after the
  // exponent (an out-of-window score may give +inf there, which the mask
  // clears before the row sum), and row sums of the bf16 probabilities.
  constexpr bool kAccMask = !(TALL && D == 64);
  f32x16 xbias;
  uint32_t xpk[8];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int p = (SEG == 16 ? ((i >> 2) & 1) * 8 : (i >> 2) * 8) + hf * 4 + (i & 3);
    const bool in = (unsigned)(p - sx) < (unsigned)kw;
    xbias[i] = in ? 0.0f : -__builtin_inff();
    if (i & 1)
      xpk[i >> 1] |= in ? 0xffff0000u : 0u;
    else
      xpk[i >> 1] = in ? 0xffffu : 0u;
  }
  const f32x16 s_init = kAccMask ? xbias : f32x16{};

  const int64_t tok_stride = (int64_t)a.NH * D;
  const int64_t head_off = (int64_t)uniform_u64((uint64_t)((int64_t)b * T * Hs * W * tok_stride + (int64_t)head * D));
  const bf16* qg = (const bf16*)a.q + head_off;
  const bf16* kg = (const bf16*)a.k + head_off;
  const bf16* vg = (const bf16*)a.v + head_off;
  bf16* og = (bf16*)a.o + head_off;
  auto token = [&](int tt, int yy, int xx) -> int64_t { return ((int64_t)tt * Hs + yy) * W + xx; };

  bf16x8 qr[C::kQK];
  {
    const bf16* p = qg + token(tqc, yqc, xqc) * tok_stride + hf * 8;
#pragma unroll
    for (int ds = 0; ds < C::kQK; ++ds) qr[ds] = *(const bf16x8*)(p + ds * 16);
  }

  // ---- DMA of one step of one tensor: copy i covers LDS row i / G of the
  // slot (G = kRowL / 1 KiB copies per row), half-plane (i % G) / (kNS/8)
  // and key slots 8*((i % G) % (kNS/8)) + 0..7; wave w issues copies w,
  // w + 4, ... The lane-dependent part of each copy's source (x position,
  // half, swizzled 16-byte chunk) is fixed for the workgroup; the row tokens
  // change per step and are scalar.
  constexpr int kGroups = C::kRowL / 1024;           // copies per LDS row
  constexpr int kGroupsPerHalf = C::kNS / C::kKeysPerCopy;
  const int srow = lane >> 3, scol = lane & 7;
  // lane byte offset from the row's first token (w * NH * D < 2^30 elements,
  // checked on the host, so it fits 31 bits); copies go through a buffer
  // resource based at the row
  uint32_t dma_voff[C::kCopiesPerWave];
  int dma_dst[C::kCopiesPerWave], dma_row[C::kCopiesPerWave];
#pragma unroll
  for (int p = 0; p < C::kCopiesPerWave; ++p) {
    const int i = min(wave + C::kWaves * p, C::kCopies - 1);
    const int g = i % kGroups;
    const int half = g / kGroupsPerHalf;
    const int pos = C::kKeysPerCopy * (g % kGroupsPerHalf) + srow;
    dma_row[p] = i / kGroups;
    dma_dst[p] = dma_row[p] * C::kRowL + g * 1024;
    dma_voff[p] =
        (uint32_t)((int64_t)min(X_lo + pos, W - 1) * tok_stride + half * 64 + ((scol ^ half_swizzle(pos)) * 8)) * 2u;
  }
  // Box rows are walked with cursors (row index, its y in the box, its token
  // offset) that advance one row at a time and stop at the last row, so no
  // step divides by NY.
  struct Cursor {
    int r, yr, tr;
    int64_t tok;
  };
  const int64_t row_step = (int64_t)W * tok_stride;             // next y
  const int64_t plane_jump = (int64_t)(Hs - NY) * W * tok_stride;  // last y of a plane -> first y of the next
  const int64_t tok0 = ((int64_t)t_lo * Hs + Y_lo) * W * tok_stride;  // the box's first row
  // Deep t windows (the t-plane-first brick order) walk their box planes
  // from the one whose t is a multiple of NT, wrapping round: bricks whose
  // boxes share a plane then read it in the same phase of their walks, while
  // its rows are in L2 (stage 5 1.609 -> 1.51 ms: per cycle the same, but
  // the chip holds a 7 % higher clock with the fabric traffic saved; at a
  // (3,7,7) window, in the launch order, 2 % slower, so the others walk
  // their planes in order).
  const int p0 = a.order == kNaOrderTColumns ? uni((NT - t_lo % NT) % NT) : 0;
  // The cursor is wave-uniform; moving it through readfirstlane keeps its
  // arithmetic on the scalar unit (left to itself the compiler walked it in
  // 64-bit vector registers: ~60 VALU instructions per step).
  auto advance = [&](Cursor& c) {
    if (c.r + 1 < nrows) {
      ++c.r;
      c.tok += row_step;
      if (++c.yr == NY) {
        c.yr = 0;
        if (c.tr + 1 == NT) {  // (a phase walk's wrap to the box's first plane)
          c.tr = 0;
          c.tok = tok0;
        } else {
          ++c.tr;
          c.tok += plane_jump;
        }
      }
    }
    c.r = __builtin_amdgcn_readfirstlane(c.r);
    c.yr = __builtin_amdgcn_readfirstlane(c.yr);
    c.tr = __builtin_amdgcn_readfirstlane(c.tr);
    c.tok = (int64_t)uniform_u64((uint64_t)c.tok);
  };
  const Cursor first = {0, 0, p0, tok0 + (int64_t)p0 * (W * (int64_t)Hs) * tok_stride};
  // The key rows of one step (their token offsets and y in the box), taken
  // from the cursor, which moves on by kRows rows. K walks the rows; V and
  // the window mask use each step's record two steps later, so only one
  // cursor runs (the scalar unit is shared by the CU's 8-16 waves).
  struct StepRows {
    int64_t tok0, tok1;
    int yr0, yr1;
    int tr0, tr1;  // (deep bricks: the rows' planes in the box)
  };
  auto next_rows = [&](Cursor& c) -> StepRows {
    StepRows rr;
    rr.tok0 = c.tok;
    rr.yr0 = c.yr;
    rr.tr0 = c.tr;
    advance(c);
    rr.tok1 = C::kRows == 2 ? c.tok : rr.tok0;
    rr.yr1 = C::kRows == 2 ? c.yr : rr.yr0;
    rr.tr1 = C::kRows == 2 ? c.tr : rr.tr0;
    if (C::kRows == 2) advance(c);
    return rr;
  };
  // Issues one tensor's copies of one step's rows. When a step's copies do
  // not divide evenly over the waves, the waves below kExtraWaves issue one
  // more. (Making that a compile-time tag of the key loop, as IN below is,
  // made the 8-wave tall kernel spill.)
  constexpr int kExtraWaves = C::kCopies % C::kWaves;
  const bool extra = kExtraWaves == 0 || wave < kExtraWaves;  // wave-uniform
  auto issue = [&](const bf16* base, int slot_off, const StepRows& rr) {
#pragma unroll
    for (int p = 0; p < C::kCopiesPerWave; ++p)
      if (kExtraWaves == 0 || p + 1 < C::kCopiesPerWave || extra)
        lds_dma16_buf(raw_rsrc(base + (dma_row[p] ? rr.tok1 : rr.tok0)), dma_voff[p], lds_base + slot_off + dma_dst[p]);
  };
  using True = std::integral_constant<bool, true>;
  using False = std::integral_constant<bool, false>;

  // ---- per-lane LDS offsets (half-plane 0; d 64-127 add kHalfL). K
  // fragment: key col of the chunk (SEG = 16: keys 0-15 from the step's first
  // row, 16-31 from its second).
  int kbase, ksw;
  if (SEG == 16) {
    const int pos = ox + (col & 15);
    kbase = (col >> 4) * C::kRowL + pos * 128;
    ksw = half_swizzle(pos);
  } else {
    const int pos = ox + col;
    kbase = pos * 128;
    ksw = half_swizzle(pos);
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
    const int sw = half_swizzle(pos);
#pragma unroll
    for (int db1 = 0; db1 < 2; ++db1)
      voff[e][db1] = pos * 128 + (((4 * db1 + 2 * dh + (vc >> 1)) ^ sw) * 16) + (vc & 1) * 8;
  }
  auto vfrag = [&](const VX_LDS unsigned char* vb, int j, int db) -> bf16x8 {
    const int jo = SEG == 16 ? j * C::kRowL : j * 16 * 128;
    const VX_LDS unsigned char* p0 = vb + jo + voff[0][db & 1] + (db >> 1) * C::kHalfL;
    const VX_LDS unsigned char* p1 = vb + jo + voff[1][db & 1] + (db >> 1) * C::kHalfL;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)p0);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)p1);
    return concat(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi));
  };
  auto kfrag = [&](const VX_LDS unsigned char* kb, int ds) -> bf16x8 {
    return *(const VX_LDS bf16x8*)(kb + koff[ds & 3] + (ds >> 2) * C::kHalfL);
  };
  constexpr int kDB = D / 32;  // 32-wide d blocks of O

  f32x16 O[kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db) O[db] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;
  const float c2 = a.scale * kLog2e;

  // ---- prologue: K of steps 0 and 1 in flight, V slot 1 zeroed (it stands
  // in for the V of step -1, paired with P = 0), S = QK^T of chunk 0.
  Cursor kcur = first;  // rows of the next K step to issue
  StepRows rows_even = next_rows(kcur), rows_odd = next_rows(kcur);  // steps 0 and 1
  issue(kg, C::kK, rows_even);
  issue(kg, C::kK + C::kSlot, rows_odd);
  for (int off = threadIdx.x * 16; off < C::kSlot; off += C::kThreads * 16)
    *(VX_LDS u32x4*)(lds + C::kV + C::kSlot + off) = u32x4{0, 0, 0, 0};
  // q preparation while the first key rows land (its loads overlap theirs)
  if (a.q_prep != 0) prep_q(qr, hf, token(tqc, yqc, xqc), tqc, yqc, xqc, a);
  wait_vmem<0>();
  __syncthreads();
  f32x16 S = s_init;
#pragma unroll
  for (int ds = 0; ds < C::kQK; ++ds) S = mfma32x32x16(kfrag(lds + C::kK, ds), qr[ds], S);
  bf16x8 Pp[2] = {bf16x8{}, bf16x8{}};

  // One step: consumes S (scores of chunk s) and Pp (probabilities of chunk
  // s-1), produces Sn (scores of chunk s+1) and P (probabilities of chunk s).
  // rr: the rows of step s on entry (their K was issued two steps ago), the
  // rows of step s + 2 on return. IN (compile-time, so that the loop carries
  // no per-step test of it): some query of this wave lies inside the grid.
  // t-stacked bricks: whether some row of chunk c (rows r) lies in this
  // wave's t window (st is the wave's first plane in the box: its lanes
  // share one t plane)
  const int st_w = C::kTStack ? uni(st) : 0;
  auto chunk_active = [&](const StepRows& r, int c) -> bool {
    if constexpr (!C::kTStack) return true;
    const int r0 = c * C::kRows;
    return (r0 < nrows && (unsigned)(r.tr0 - st_w) < (unsigned)kt) ||
           (r0 + 1 < nrows && (unsigned)(r.tr1 - st_w) < (unsigned)kt);
  };
  auto step = [&](auto in_tag, const int s, f32x16& S, f32x16& Sn, const bf16x8 (&Pp)[2], bf16x8 (&P)[2],
                  StepRows& rr, const StepRows& rn, bool& act_prev) __attribute__((always_inline)) {
    constexpr bool IN = decltype(in_tag)::value;
    // (t-stacked bricks) chunk s's rows are rr's on entry, chunk s+1's rn's
    const bool act_cur = chunk_active(rr, s), act_next = chunk_active(rn, s + 1);
    const bool idle = C::kTStack && !act_prev && !act_cur && !act_next;
    // The previous step's copies (K of s+1, V of s-1) have landed once this
    // wave has none outstanding; the barrier publishes everyone's and frees
    // K slot s%2 (K of s, read last step) and V slot s%2 (V of s-2).
    wait_vmem<0>();
    __syncthreads();
    // y window of chunk s: whether each of its key rows lies in this lane's
    // window (the x window is in the scores already, as -inf)
    bool row_ok[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int r = s * C::kRows + (SEG == 16 ? h2 : 0);
      row_ok[h2] = r < nrows && (unsigned)((h2 == 0 ? rr.yr0 : rr.yr1) - sy) < (unsigned)kh &&
                   (C::kQT == 1 || (unsigned)((h2 == 0 ? rr.tr0 : rr.tr1) - st) < (unsigned)kt);
    }
    const StepRows cur = rr;
    rr = next_rows(kcur);
    // This wave's copies of the step, V of step s (copies 0 .. kCopiesPerWave-1)
    // then K of step s + 2: copy j is issued in MFMA slot j, so that a wave's
    // matrix and softmax work does not queue behind its copies (a wave issues
    // in order, and the CU's load path takes each 1 KiB copy in ~16 cycles).
    auto copy = [&](int j) __attribute__((always_inline)) {
      const bool isv = j < C::kCopiesPerWave;
      const int p = isv ? j : j - C::kCopiesPerWave;
      if (kExtraWaves == 0 || p + 1 < C::kCopiesPerWave || extra) {
        const StepRows& r = isv ? cur : rr;
        lds_dma16_buf(raw_rsrc((isv ? vg : kg) + (dma_row[p] ? r.tok1 : r.tok0)), dma_voff[p],
                      lds_base + (isv ? C::kV : C::kK) + (s & 1) * C::kSlot + dma_dst[p]);
      }
    };
    constexpr int kStepCopies = 2 * C::kCopiesPerWave;
    static_assert(kStepCopies <= C::kSlots, "one copy per MFMA slot at most");

    const VX_LDS unsigned char* kb = lds + C::kK + ((s + 1) & 1) * C::kSlot;  // K of chunk s+1
    const VX_LDS unsigned char* vb = lds + C::kV + ((s + 1) & 1) * C::kSlot;  // V of chunk s-1
    // (IN is the tag's value; the 1 x 4 x 32 bricks pass the runtime flag
    // instead, one loop for all waves: their two loops measured ~1 % slower
    // at the (3,7,7) config, whose x edge holds waves without queries)
    if (!(IN && (TALL || wave_in)) || idle) {
      // no query of this wave is inside the grid (the ragged x or y edge),
      // or (t-stacked bricks) none of chunks s-1, s, s+1 has a row in its t
      // window: it only copies its share of the rows. An idle step's chunk
      // s+1 scores start from the x window alone (no row of it counts).
#pragma unroll
      for (int j = 0; j < kStepCopies; ++j) copy(j);
      P[0] = bf16x8{};
      P[1] = bf16x8{};
      if (idle) Sn = s_init;
      act_prev = act_cur;
      return;
    }
    // PV fragment f < kPV: key half j = f / kDB, d block f % kDB; then QK^T.
    auto frag = [&](int i) -> bf16x8 {
      return i < C::kPV ? vfrag(vb, i / kDB, i % kDB) : kfrag(kb, i - C::kPV);
    };
    Sn = s_init;
    // exponent offset per key row: -m_run, or -inf for a row outside the y
    // window (exp2 then gives 0)
    const float mrow[2] = {row_ok[0] ? -m_run : -__builtin_inff(), row_ok[1] ? -m_run : -__builtin_inff()};
    const bf16x2 one2 = {(bf16)1.0f, (bf16)1.0f};
    float l_tile = 0.f;
    bf16x8 fr[C::kSlots];
    float pf[16];
    // wave priority 1 while in the slots, ahead of the other workgroup's
    // wave on the SIMD while that one copies or waits (+1.5-2.5 % with the
    // tall bricks, neutral with (3,7,7) windows)
    __builtin_amdgcn_s_setprio(1);
    bf16x2 pk[8];
    fr[0] = frag(0);
    fr[1] = frag(1);
    // kSlots slots: slot i issues one MFMA (i < kPV: PV(s-1), else QK^T(s+1)),
    // the LDS read two slots ahead, and the mask + exp of kScoresPerSlot
    // scores of chunk s.
    if constexpr (TALL && D == 64) {
      // tall bricks at head dim 64: the MFMA block, then the masking and
      // softmax block, so the two waves of a SIMD alternate between them
      // (+1.6 % at the (11, 11, 11) window; at head dim 128 and in the
      // 1 x 4 x 32 bricks the per-slot interleave measured as fast or faster)
#pragma unroll
      for (int i = 0; i < C::kSlots; ++i) {
        if (i + 2 < C::kSlots) fr[i + 2] = frag(i + 2);
        if (i < C::kPV)
          O[i % kDB] = mfma32x32x16(fr[i], Pp[i / kDB], O[i % kDB]);
        else
          Sn = mfma32x32x16(fr[i], qr[i - C::kPV], Sn);
        if (i < kStepCopies) copy(i);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[8 * g + i] = __builtin_fmaf(S[8 * g + i], c2, mrow[g]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[8 * g + i] = fast_exp2(pf[8 * g + i]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // (the tall D = 64 block: kAccMask is false, the x window is xpk)
          const bf16x2 pr = bf16x2{(bf16)pf[8 * g + 2 * i], (bf16)pf[8 * g + 2 * i + 1]};
          pk[4 * g + i] = __builtin_bit_cast(bf16x2, __builtin_bit_cast(uint32_t, pr) & xpk[4 * g + i]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // row sums of the bf16 probabilities (dot2 with 1, 1): fp32 sums of
      // the unrounded ones keep pf live past the packing, 5 spills at 128 VGPRs
      l_tile = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) l_tile = __builtin_amdgcn_fdot2_f32_bf16(pk[i], one2, l_tile, false);
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int i = 0; i < C::kSlots; ++i) {
        if (i + 2 < C::kSlots) fr[i + 2] = frag(i + 2);
        if (i < C::kPV)
          O[i % kDB] = mfma32x32x16(fr[i], Pp[i / kDB], O[i % kDB]);
        else
          Sn = mfma32x32x16(fr[i], qr[i - C::kPV], Sn);
        if (i < kStepCopies) copy(i);
#pragma unroll
        for (int u = 0; u < C::kScoresPerSlot; ++u) {
          const int e = i * C::kScoresPerSlot + u;
          static_assert(kAccMask, "the per-slot form runs with the accumulator-start x window");
          pf[e] = fast_exp2(__builtin_fmaf(S[e], c2, mrow[e >> 3]));
          if (e & 1) pk[e >> 1] = bf16x2{(bf16)pf[e - 1], (bf16)pf[e]};
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      l_tile = sum16(pf);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      P[j] = __builtin_shufflevector(__builtin_shufflevector(pk[4 * j], pk[4 * j + 1], 0, 1, 2, 3),
                                     __builtin_shufflevector(pk[4 * j + 2], pk[4 * j + 3], 0, 1, 2, 3),
                                     0, 1, 2, 3, 4, 5, 6, 7);
    __builtin_amdgcn_s_setprio(0);
    // rare: a probability may exceed 2^kRescaleSlack (the lane's chunk sum is
    // above kSumLimit, inf or NaN; the first chunk with a key in the window
    // always lands here) -> raise m_run to the chunk max, rescale O and l and
    // recompute the chunk's probabilities.
    if (__builtin_amdgcn_ballot_w64(l_tile > kSumLimit || is_nan_bits(l_tile)) != 0) {
      // (with kAccMask the scores carry the x window; without it xpk holds it)
      float mx = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bool in = row_ok[i >> 3] && (kAccMask || ((xpk[i >> 1] >> ((i & 1) * 16)) & 1u) != 0);
        mx = __builtin_fmaxf(mx, in ? S[i] : -__builtin_inff());
      }
      const float mn = __builtin_fmaxf(m_run, halves_max(mx) * c2);
      const float alpha = fast_exp2(m_run - mn);
      m_run = mn;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < kDB; ++db) O[db] *= alpha;
      if constexpr (kAccMask) {
        const float mr[2] = {row_ok[0] ? -mn : -__builtin_inff(), row_ok[1] ? -mn : -__builtin_inff()};
#pragma unroll
        for (int e = 0; e < 16; ++e) pf[e] = fast_exp2(__builtin_fmaf(S[e], c2, mr[e >> 3]));
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          bf16x8 pv;
#pragma unroll
          for (int r = 0; r < 8; ++r) pv[r] = (bf16)pf[8 * j + r];
          P[j] = pv;
        }
        l_tile = sum16(pf);
      } else {
        const float mr[2] = {row_ok[0] ? -mn : -__builtin_inff(), row_ok[1] ? -mn : -__builtin_inff()};
        l_tile = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          bf16x8 pv;
#pragma unroll
          for (int r = 0; r < 8; ++r) pv[r] = (bf16)fast_exp2(__builtin_fmaf(S[8 * j + r], c2, mr[j]));
          u32x4 w = __builtin_bit_cast(u32x4, pv);
#pragma unroll
          for (int q = 0; q < 4; ++q) w[q] &= xpk[4 * j + q];
          pv = __builtin_bit_cast(bf16x8, w);
          P[j] = pv;
          l_tile = sum8(pv, l_tile);
        }
      }
    }
    l_run += l_tile;
    act_prev = act_cur;
  };

  f32x16 S2;
  bf16x8 P2[2];
  // the key loop; the tall bricks run one copy for the waves with queries
  // and one for the others
  bool act_prev = false;  // chunk -1 (none)
  auto key_loop = [&](auto in_tag) __attribute__((always_inline)) {
    int s = 0;
    for (; s + 1 < n_steps; s += 2) {
      step(in_tag, s, S, S2, Pp, P2, rows_even, rows_odd, act_prev);
      step(in_tag, s + 1, S2, S, P2, Pp, rows_odd, rows_even, act_prev);
    }
    if (s < n_steps) {
      step(in_tag, s, S, S2, Pp, P2, rows_even, rows_odd, act_prev);
      Pp[0] = P2[0];
      Pp[1] = P2[1];
    }
  };
  if (!TALL || wave_in)
    key_loop(True{});
  else
    key_loop(False{});
  // ---- PV of the last chunk (its V was issued by the last step).
  wait_vmem<0>();
  __syncthreads();
  {
    const VX_LDS unsigned char* vb = lds + C::kV + ((n_steps - 1) & 1) * C::kSlot;
#pragma unroll
    for (int i = 0; i < C::kPV; ++i) O[i % kDB] = mfma32x32x16(vfrag(vb, i / kDB, i % kDB), Pp[i / kDB], O[i % kDB]);
  }

  const float lt = halves_sum(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  store_na_rows<kDB, C::kQX, C::kQY>(O, inv, og, tok_stride, tw, y0, xq0, T, Hs, W, lane);
}

// Three waves per SIMD for the 32-key segments at head dim 64 (146 VGPRs,
// three 32 KiB workgroups per CU): 33x88x160 NH=4 at a (5,5,21) window
// 1.02 -> 0.94 ms. The 16-key form gained at 21x45x80 NH=24 (-9 %) but lost
// at 33x88x160 NH=4 (+3.5 %) and keeps two.
template <int SEG, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 64 && SEG == 32 ? 3 : 2,
                                                                       D == 64 && SEG == 32 ? 3 : 2)))
void na3d_pipe_kernel(const Na3dArgs a, int n_yb, int n_xb) {
  na3d_pipe_body<SEG, D, false>(a, n_yb, n_xb);
}

// Head dim 64: four waves per SIMD (at most 128 VGPRs; the workgroup's 32 KiB
// of LDS allows four per CU), so that more workgroups cover each other's
// per-step waits: 2.56 -> 2.31 ms at the (11, 11, 11) window on 33x88x160.
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 64 ? 4 : 2, D == 64 ? 4 : 2)))
void na3d_tall_kernel(const Na3dArgs a, int n_yb, int n_xb) {
  na3d_pipe_body<16, D, true>(a, n_yb, n_xb);
}

// Head dim 64, grids whose width rounds up to the same multiple of 16 and 32
// (no more ragged columns than the narrow bricks): 1 x 8 x 32 bricks of 8
// waves, two workgroups of 48 KiB per CU. 33x88x160: 2.31 -> 2.09 ms.
template <int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4)))
void na3d_tall_wide_kernel(const Na3dArgs a, int n_yb, int n_xb) {
  na3d_pipe_body<16, D, true, true>(a, n_yb, n_xb);
}

// Head dim 64, deep t windows: the wide bricks two t planes deep (2 x 4 x 32,
// waves of 2 t x 4 y x 4 x), two workgroups of 48 KiB per CU.
template <int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4)))
void na3d_deep_kernel(const Na3dArgs a, int n_yb, int n_xb) {
  na3d_pipe_body<16, D, true, true, true>(a, n_yb, n_xb);
}

// Head dim 128, windows up to 9 wide and t windows of 2 and more: the
// t-stacked 2 x 4 x 16 bricks, two workgroups of 48 KiB per CU.
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void na3d_tstack_kernel(const Na3dArgs a, int n_yb, int n_xb) {
  na3d_pipe_body<16, D, false, false, false, true>(a, n_yb, n_xb);
}

}  // namespace

int launch_na3d_fwd(const Na3dArgs& a, void* stream, const char** launched) {
  if (a.D != 128 && a.D != 64) return (int)hipErrorNotSupported;
  hipStream_t st = (hipStream_t)stream;
  switch (a.variant) {
    case kNaTall: {
      const int n_yb = (a.Hs + 7) / 8;
      const int n_xb = (a.W + 15) / 16;
      dim3 grid((unsigned)a.T * n_yb * n_xb, a.NH, a.B);
      if (a.D == 128) {
        hipLaunchKernelGGL((na3d_tall_kernel<128>), grid, dim3(256), 0, st, a, n_yb, n_xb);
        *launched = "na3d_tall_kernel<128>";
      } else {
        hipLaunchKernelGGL((na3d_tall_kernel<64>), grid, dim3(256), 0, st, a, n_yb, n_xb);
        *launched = "na3d_tall_kernel<64>";
      }
      return (int)hipGetLastError();
    }
    case kNaTallWide: {
      if (a.D != 64) return (int)hipErrorNotSupported;
      const int n_yb = (a.Hs + 7) / 8;
      const int n_xb = (a.W + 31) / 32;
      dim3 grid((unsigned)a.T * n_yb * n_xb, a.NH, a.B);
      hipLaunchKernelGGL((na3d_tall_wide_kernel<64>), grid, dim3(512), 0, st, a, n_yb, n_xb);
      *launched = "na3d_tall_wide_kernel<64>";
      return (int)hipGetLastError();
    }
    case kNaDeep: {
      if (a.D != 64) return (int)hipErrorNotSupported;
      const int n_yb = (a.Hs + 3) / 4;
      const int n_xb = (a.W + 31) / 32;
      dim3 grid((unsigned)((a.T + 1) / 2) * n_yb * n_xb, a.NH, a.B);
      hipLaunchKernelGGL((na3d_deep_kernel<64>), grid, dim3(512), 0, st, a, n_yb, n_xb);
      *launched = "na3d_deep_kernel<64>";
      return (int)hipGetLastError();
    }
    case kNaTStack: {
      if (a.D != 128) return (int)hipErrorNotSupported;
      const int n_yb = (a.Hs + 3) / 4;
      const int n_xb = (a.W + 15) / 16;
      dim3 grid((unsigned)((a.T + 1) / 2) * n_yb * n_xb, a.NH, a.B);
      hipLaunchKernelGGL((na3d_tstack_kernel<128>), grid, dim3(256), 0, st, a, n_yb, n_xb);
      *launched = "na3d_tstack_kernel<128>";
      return (int)hipGetLastError();
    }
    case kNaPipe16:
    case kNaPipe32: {
      const int n_yb = (a.Hs + 3) / 4;
      const int n_xb = (a.W + 31) / 32;
      dim3 grid((unsigned)a.T * n_yb * n_xb, a.NH, a.B);
      if (a.variant == kNaPipe16 && a.D == 128) {
        hipLaunchKernelGGL((na3d_pipe_kernel<16, 128>), grid, dim3(256), 0, st, a, n_yb, n_xb);
        *launched = "na3d_pipe_kernel<16, 128>";
      } else if (a.D == 128) {
        hipLaunchKernelGGL((na3d_pipe_kernel<32, 128>), grid, dim3(256), 0, st, a, n_yb, n_xb);
        *launched = "na3d_pipe_kernel<32, 128>";
      } else if (a.variant == kNaPipe16) {
        hipLaunchKernelGGL((na3d_pipe_kernel<16, 64>), grid, dim3(256), 0, st, a, n_yb, n_xb);
        *launched = "na3d_pipe_kernel<16, 64>";
      } else {
        hipLaunchKernelGGL((na3d_pipe_kernel<32, 64>), grid, dim3(256), 0, st, a, n_yb, n_xb);
        *launched = "na3d_pipe_kernel<32, 64>";
      }
      return (int)hipGetLastError();
    }
    case kNaWave: {
      const int n_yb = (a.Hs + kBrickY - 1) / kBrickY;
      const int n_xb = (a.W + kBrickX - 1) / kBrickX;
      const int n_xg = (n_xb + kWaves - 1) / kWaves;
      dim3 grid((unsigned)a.T * n_yb * n_xg, a.NH, a.B);
      if (a.D == 128) {
        hipLaunchKernelGGL((na3d_wave_kernel<128>), grid, dim3(kWaves * 64), 0, st, a, n_yb, n_xb, n_xg);
        *launched = "na3d_wave_kernel<128>";
      } else {
        hipLaunchKernelGGL((na3d_wave_kernel<64>), grid, dim3(kWaves * 64), 0, st, a, n_yb, n_xb, n_xg);
        *launched = "na3d_wave_kernel<64>";
      }
      return (int)hipGetLastError();
    }
    default:
      return (int)hipErrorInvalidValue;
  }
}

}  // namespace vx
