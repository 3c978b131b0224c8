// Non-causal flash attention forward for gfx950, bf16 in/out, D = 128.
//
// Work decomposition: one workgroup per (query tile, head, batch); WAVES
// waves per workgroup, each owning NQB blocks of 32 query rows. The wave
// computes S^T = K Q^T so that every lane owns one query column of the MFMA
// output: row max, row sum and the output rescale are per-lane scalars and the
// two halves of the wave are combined with one v_permlane32_swap. Q stays in
// registers as the B operand for the whole key loop. K and V tiles of 64 keys
// are staged through registers into double-buffered, XOR-swizzled LDS; K is
// read back with ds_read_b128 (A operand of QK^T) and V with the gfx950
// transpose read ds_read_b64_tr_b16 (A operand of O^T = V^T P^T). The QK^T of
// tile t+1 is issued before the softmax of tile t so the matrix cores and
// the VALU overlap within a wave.
//
// Softmax: scores are kept in log2 units (scale * log2(e) folded into one
// FMA before v_exp_f32). The running row max is only raised when a tile's
// max exceeds it by more than kRescaleSlack (log2 units), which bounds the
// unnormalised probabilities by 2^kRescaleSlack and makes the O rescale rare;
// the final division by the row sum makes the result independent of the
// reference point.
#include "vx_gfx950.hpp"
#include "vx_kernels.h"

namespace vx {
namespace {

constexpr int kD = 128;
constexpr int kBN = 64;                       // keys per tile
constexpr int kRowBytes = kD * 2;             // one bf16 key row
constexpr int kTileBytes = kBN * kRowBytes;   // 16 KiB
constexpr float kRescaleSlack = 8.0f;         // log2 units
constexpr float kNegBig = -1.0e30f;           // finite "no key seen yet" max

// XOR swizzle of the 16-byte chunk index within a 256-byte LDS row. Eight
// consecutive rows map one chunk to eight distinct 16-byte bank groups (the
// ds_read_b128 K reads), and rows 4i..4i+3 map a chunk pair to four distinct
// pairs (the transpose reads of V).
__device__ __forceinline__ int row_swizzle(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

template <int NQB, int WAVES, bool MASKED>
struct FlashTile {
  static constexpr int kThreads = WAVES * 64;
  static constexpr int kQueriesPerWave = NQB * 32;
  static constexpr int kQueriesPerBlock = WAVES * kQueriesPerWave;
  static constexpr int kLoadsPerWave = (kBN / 4) / WAVES;  // 1 KiB wave loads per tile
  static_assert(kLoadsPerWave >= 1, "too many waves for one tile");
};

template <int NQB, int WAVES, bool MASKED>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WAVES / 4, WAVES / 4)))
void flash_fwd_kernel(const FlashArgs a) {
  using T = FlashTile<NQB, WAVES, MASKED>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[4 * kTileBytes];
  unsigned char* const kbuf0 = smem;
  unsigned char* const kbuf1 = smem + kTileBytes;
  unsigned char* const vbuf0 = smem + 2 * kTileBytes;
  unsigned char* const vbuf1 = smem + 3 * kTileBytes;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hf = lane >> 5;   // which half of the wave
  const int col = lane & 31;  // query column within a 32-block
  const int b = blockIdx.z;
  const int head = blockIdx.y;
  const int qw0 = (blockIdx.x * WAVES + wave) * T::kQueriesPerWave;

  const bf16* qg = (const bf16*)a.q + b * a.qs[0] + head * a.qs[2];
  const bf16* kg = (const bf16*)a.k + b * a.ks[0] + head * a.ks[2];
  const bf16* vg = (const bf16*)a.v + b * a.vs[0] + head * a.vs[2];
  bf16* og = (bf16*)a.o + b * a.os[0] + head * a.os[2];

  int kv_end = a.Sk;
  if (a.kv_len != nullptr) kv_end = min(max(a.kv_len[b], 0), a.Sk);
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  const float c = a.scale * kLog2e;

  // ---- Q (B operand of S^T = K Q^T), resident for the whole key loop.
  bf16x8 qr[NQB][8];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int qi = min(qw0 + qb * 32 + col, a.Sq - 1);
    const bf16* p = qg + (int64_t)qi * a.qs[1] + hf * 8;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) qr[qb][ds] = *(const bf16x8*)(p + ds * 16);
  }

  // ---- per-lane LDS offsets.
  // K fragment (kb, ds): row kb*32 + col, chunk 2*ds + hf, swizzled by row%8 = col%8.
  const int ksw = row_swizzle(col);
  int koff[4];
#pragma unroll
  for (int d4 = 0; d4 < 4; ++d4) koff[d4] = col * kRowBytes + (((2 * d4 + hf) ^ ksw) * 16);
  // V transpose read (kb, j, db, e): group g = lane/16 covers columns
  // db*32 + (g%2)*16 + 0..15 of rows kb*32 + 16j + 8e + hf*4 + 0..3.
  const int i16 = lane & 15;
  const int vr = i16 >> 2, vc = i16 & 3, dh = (lane >> 4) & 1;
  const int vsw = 2 * vr + hf;  // row_swizzle of those rows
  int voff[2];
#pragma unroll
  for (int db1 = 0; db1 < 2; ++db1)
    voff[db1] = (hf * 4 + vr) * kRowBytes + (((4 * db1 + 2 * dh + (vc >> 1)) ^ vsw) * 16) + (vc & 1) * 8;

  // ---- global -> register -> LDS staging of one 64-key tile.
  u32x4 kst[T::kLoadsPerWave], vst[T::kLoadsPerWave];
  auto gload = [&](const bf16* base, int64_t sstride, int t, u32x4* st) {
#pragma unroll
    for (int p = 0; p < T::kLoadsPerWave; ++p) {
      const int r = (wave * T::kLoadsPerWave + p) * 4 + (lane >> 4);
      const int key = min(t * kBN + r, kv_end - 1);
      st[p] = *(const u32x4*)(base + (int64_t)key * sstride + (lane & 15) * 8);
    }
  };
  auto lstore = [&](unsigned char* buf, const u32x4* st) {
#pragma unroll
    for (int p = 0; p < T::kLoadsPerWave; ++p) {
      const int r = (wave * T::kLoadsPerWave + p) * 4 + (lane >> 4);
      const int pos = (lane & 15) ^ row_swizzle(r);
      *(u32x4*)(buf + r * kRowBytes + pos * 16) = st[p];
    }
  };

  auto qk = [&](const unsigned char* buf, f32x16 (&S)[2][NQB]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) S[kb][qb] = f32x16{};
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 kf =
            *(const bf16x8*)(buf + kb * 32 * kRowBytes + (ds >> 2) * 128 + koff[ds & 3]);
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) S[kb][qb] = mfma32x32x16(kf, qr[qb][ds], S[kb][qb]);
      }
    }
  };

  f32x16 O[4][NQB];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) O[db][qb] = f32x16{};
  float m_run[NQB], l_run[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m_run[qb] = kNegBig;
    l_run[qb] = 0.f;
  }

  const uint8_t* vrow = (MASKED && a.key_valid) ? a.key_valid + (int64_t)b * a.key_mask_stride : nullptr;
  const float* brow = (MASKED && a.key_bias) ? a.key_bias + (int64_t)b * a.key_mask_stride : nullptr;

  if (n_tiles > 0) {
    // Prologue: K0, V0 and K1 into LDS, then S(0).
    gload(kg, a.ks[1], 0, kst);
    gload(vg, a.vs[1], 0, vst);
    lstore(kbuf0, kst);
    lstore(vbuf0, vst);
    if (n_tiles > 1) {
      gload(kg, a.ks[1], 1, kst);
      lstore(kbuf1, kst);
    }
    __syncthreads();
    f32x16 S[2][NQB];
    qk(kbuf0, S);

    for (int t = 0; t < n_tiles; ++t) {
      // LDS now holds K_{t+1} in kbuf[(t+1)%2] and V_t in vbuf[t%2].
      __syncthreads();
      const bool has_next = t + 1 < n_tiles;
      if (t + 2 < n_tiles) gload(kg, a.ks[1], t + 2, kst);
      if (has_next) gload(vg, a.vs[1], t + 1, vst);

      f32x16 Sn[2][NQB];
      if (has_next) qk((t & 1) ? kbuf0 : kbuf1, Sn);

      // ---- key masks. Tiles that hold a masked key (the tail tile, a
      // key_valid hole, any key_bias) take the scores to log2 units here,
      // masked keys -> -inf, and use cc = 1 below; fully valid tiles keep the
      // fused scale in the exp argument.
      const int key0 = t * kBN;
      const int klast = (kv_end - 1) & ~3;  // last aligned 4-key group inside the loop
      uint32_t vbits[2][4];
      bool slow = key0 + kBN > kv_end;
      if (MASKED) {
        if (vrow != nullptr) {
          bool hole = false;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int kbase = key0 + kb * 32 + g * 8 + hf * 4;  // multiple of 4
              vbits[kb][g] = *(const uint32_t*)(vrow + min(kbase, klast));
              // a zero byte anywhere in the word marks an invalid key
              hole |= ((vbits[kb][g] - 0x01010101u) & ~vbits[kb][g] & 0x80808080u) != 0;
            }
          slow = slow || __builtin_amdgcn_ballot_w64(hole) != 0;
        }
        slow = slow || brow != nullptr;
      }
      float cc = c;
      if (slow) {
        cc = 1.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int kbase = key0 + kb * 32 + g * 8 + hf * 4;
            f32x4 bias = {0.f, 0.f, 0.f, 0.f};
            if (MASKED && brow != nullptr) bias = *(const f32x4*)(brow + min(kbase, klast)) * kLog2e;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              bool ok = kbase + e < kv_end;
              if (MASKED && vrow != nullptr) ok = ok && ((vbits[kb][g] >> (8 * e)) & 0xffu) != 0;
#pragma unroll
              for (int qb = 0; qb < NQB; ++qb) {
                const float sv = __builtin_fmaf(S[kb][qb][g * 4 + e], c, bias[e]);
                S[kb][qb][g * 4 + e] = ok ? sv : -__builtin_inff();
              }
            }
          }
        }
      }

      // ---- online softmax with lazy rescale.
      float ms[NQB];
      bool need = false;
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        float mx = S[0][qb][0];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, S[kb][qb][i]);
        ms[qb] = halves_max(mx) * cc;
        need |= ms[qb] > m_run[qb] + kRescaleSlack;
      }
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          const float mn = fmaxf(m_run[qb], ms[qb]);
          const float alpha = fast_exp2(m_run[qb] - mn);
          m_run[qb] = mn;
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < 4; ++db) O[db][qb] *= alpha;
        }
      }
      bf16x8 P[2][2][NQB];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        const float mneg = -m_run[qb];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            bf16x8 pv;
#pragma unroll
            for (int r = 0; r < 8; ++r)
              pv[r] = (bf16)fast_exp2(__builtin_fmaf(S[kb][qb][8 * j + r], cc, mneg));
            P[kb][j][qb] = pv;
            l_run[qb] = sum8(pv, l_run[qb]);
          }
      }

      // ---- O^T += V^T P^T.
      const unsigned char* vb = (t & 1) ? vbuf1 : vbuf0;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const unsigned char* base = vb + (kb * 32 + 16 * j) * kRowBytes + (db >> 1) * 128 + voff[db & 1];
            const bf16x8 vf = concat(lds_read_tr16(base), lds_read_tr16(base + 8 * kRowBytes));
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) O[db][qb] = mfma32x32x16(vf, P[kb][j][qb], O[db][qb]);
          }

      // ---- publish the prefetched tiles (read by everyone after the next barrier).
      if (t + 2 < n_tiles) lstore((t & 1) ? kbuf1 : kbuf0, kst);
      if (has_next) lstore((t & 1) ? vbuf0 : vbuf1, vst);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) S[kb][qb] = Sn[kb][qb];
    }
  }

  // ---- epilogue: normalise and store (lane holds 4 consecutive d per group).
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const float lt = halves_sum(l_run[qb]);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    const int qi = qw0 + qb * 32 + col;
    if (qi < a.Sq) {
      bf16* orow = og + (int64_t)qi * a.os[1];
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          bf16x4 ov;
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[e] = (bf16)(O[db][qb][g * 4 + e] * inv);
          *(bf16x4*)(orow + db * 32 + g * 8 + hf * 4) = ov;
        }
    }
  }
}

template <int NQB, int WAVES, bool MASKED>
int launch(const FlashArgs& a, hipStream_t stream) {
  using T = FlashTile<NQB, WAVES, MASKED>;
  dim3 grid((a.Sq + T::kQueriesPerBlock - 1) / T::kQueriesPerBlock, a.H, a.B);
  hipLaunchKernelGGL((flash_fwd_kernel<NQB, WAVES, MASKED>), grid, dim3(T::kThreads), 0, stream, a);
  return (int)hipGetLastError();
}

}  // namespace

int launch_flash_fwd(const FlashArgs& a, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (a.key_valid != nullptr || a.key_bias != nullptr) return launch<1, 8, true>(a, s);
  return launch<1, 8, false>(a, s);
}

}  // namespace vx
