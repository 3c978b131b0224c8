// Non-causal flash attention forward for gfx950, bf16 in/out, D = 128 or 64.
//
// Work decomposition: one workgroup of 8 waves per (256-query tile, head,
// batch item), or of 4 waves per 128-query tile for short key sequences and
// small grids (two workgroups per CU); each wave owns 32 query rows, two
// waves per SIMD. The wave
// computes S^T = K Q^T so that every lane owns one query column of the MFMA
// output: row max, row sum and the output rescale are per-lane scalars and the
// two halves of the wave are combined with one v_permlane32_swap. Q stays in
// registers as the B operand for the whole key loop. K and V tiles of 64 keys
// are copied by the LDS DMA path (buffer_load_dwordx4 ... lds, issued by
// waves 0-3) into XOR-swizzled LDS, three buffers each issued two iterations
// ahead of their use (two buffers, one iteration ahead, in 4-wave
// workgroups), so their HBM / L2 latency stays off the critical path; K is
// read back with ds_read_b128 (A operand of QK^T) and V with the gfx950
// transpose read ds_read_b64_tr_b16 (A operand of O^T = V^T P^T).
//
// Software pipeline: iteration t issues the MFMAs of QK^T(t+1) and of
// PV(t-1) in one branch-free block of 32 slots (one MFMA and the LDS read
// three slots ahead per slot, fenced with sched_barrier), and the softmax of
// tile t as a separate VALU block, so that the two waves of a SIMD alternate:
// one wave's MFMA block runs beside the other wave's softmax block.
//
// Softmax: scores are kept in log2 units (scale * log2(e) folded into the FMA
// that feeds v_exp_f32). The probabilities of a tile are computed
// speculatively against the running reference point m_run, with no max pass
// over the scores: if any probability exceeded 2^kRescaleSlack the lane's
// partial sum of the tile exceeds kSumLimit = 2^kRescaleSlack (or is inf /
// NaN), and only then is the tile max taken, m_run raised to it, O and l
// rescaled and the tile's probabilities recomputed. Every probability that is
// accumulated is therefore at most 2^kRescaleSlack. The final division by the
// row sum makes the result independent of the reference point.
#include "vx_gfx950.hpp"
#include "vx_kernels.h"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

namespace vx {
namespace {

constexpr int kBN = 64;                       // keys per tile

// Per head dim (128 or 64) and workgroup size: LDS rows, tiles, buffers and
// DMA copies. 8 waves (256 queries) keep three K and three V tiles (one
// workgroup per CU, copies issued two iterations ahead); 4 waves (128
// queries) keep two of each, so that two workgroups share a CU and hide each
// other's start (q load, pipeline fill) and end, which dominate short key
// sequences and small grids.
template <int D, int WAVES>
struct FCfg {
  static constexpr int kWaves = WAVES;
  static constexpr int kThreads = WAVES * 64;
  static constexpr int kQueriesPerBlock = WAVES * 32;
  static constexpr int kNB = WAVES == 8 ? 3 : 2;        // K (and V) tiles in LDS
  static constexpr int kRowBytes = D * 2;               // one bf16 key row
  static constexpr int kTileBytes = kBN * kRowBytes;    // 16 (8) KiB
  static constexpr int kVBuf = 0;                       // kNB V tiles
  static constexpr int kKBuf = kNB * kTileBytes;        // kNB K tiles
  static constexpr int kSmemBytes = 2 * kNB * kTileBytes;
  static constexpr int kMaskBuf = kSmemBytes;           // then the mask ring
  // In LDS a tile is D/64 half-planes of 64 keys x 128 bytes (d 0-63, then
  // d 64-127): one 1 KiB DMA copy fills 8 keys of one half-plane.
  static constexpr int kHalfBytes = kBN * 128;          // 8 KiB
  // Waves 0 .. kCopyWaves-1 issue the tile copies, kLoadsPerWave each. A
  // copy instruction holds its wave's issue for tens of cycles; with 8 waves
  // only waves 0-3 (one per SIMD) copy, so each SIMD's other wave keeps the
  // matrix core busy meanwhile.
  static constexpr int kCopyWaves = WAVES == 8 ? 4 : WAVES;
  static constexpr int kLoadsPerWave = kTileBytes / (kCopyWaves * 1024);
  static constexpr int kDB = D / 32;                    // 32-wide d blocks of O
  static constexpr int kDS = D / 16;                    // 16-deep d steps of QK^T
  static constexpr int kPV = 2 * 2 * kDB;               // MFMAs of PV per tile
  static constexpr int kQK = 2 * kDS;                   // MFMAs of QK^T per tile
  static constexpr int kSlots = kPV + kQK;              // 32 (16)
  // key masks: tile j's mask in slot j % kMaskRing. Masks are staged one
  // tile further ahead than K (tile t + kNB + 1 in iteration t), so the
  // ring holds the kNB + 1 masks in flight plus the two being read (tile
  // t's and tile t + 1's).
  static constexpr int kMaskRing = 8;
  static_assert(kNB + 3 <= kMaskRing, "mask ring too small");
};
// Key masks of the masked variants go through LDS like K: a ring of slots
// of 320 bytes (64 validity bytes, then 64 fp32 biases), staged by wave 0
// with the K copies, one tile ahead of K.
constexpr int kMaskSlot = 320;
// Mask kinds (template argument, bits): validity bytes per key, additive bias
// per key, additive bias per (query, key) of each head (read per query row
// straight from global memory: meant for the short sequences that use it).
constexpr int kMaskNone = 0, kMaskValid = 1, kMaskBias = 2, kMaskFull = 4;
constexpr float kRescaleSlack = 8.0f;         // log2 units
constexpr float kSumLimit = 256.0f;           // 2^kRescaleSlack
static_assert(kSumLimit == (float)(1 << (int)kRescaleSlack), "the tile-sum limit is 2^slack");
constexpr float kNegBig = -1.0e30f;           // finite "no key seen yet" max

typedef VX_LDS unsigned char lds_u8;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Stores a wave's 32 output rows (query rows q0 .. q0 + 31 of the head's
// output, rows at or past Sq dropped): the O^T accumulators normalised by
// inv and packed (pack_out_rows), one 64-wide d pair at a time (few
// registers), as whole 128-byte lines (line_chunks).
template <int kDB>
__device__ __forceinline__ void store_out_lines(const f32x16 (&O)[kDB], float inv, bf16* obase, int q0, int Sq,
                                                int64_t os1, int lane) {
  const int r8 = lane & 7;
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
      const int q = q0 + r8 + 8 * i;
      if (q < Sq) *(u32x4*)((unsigned char*)(obase + (int64_t)q * os1) + cofs) = out[i];
    }
  }
}

// One workgroup's work: query tile `qtile` of (head, b) over the keys
// [k_lo, k_hi) (k_lo a multiple of the key tile). part < 0 writes the
// normalised bf16 output rows; part >= 0 writes the unnormalised fp32
// accumulators, the reference point and the row sums to partial slot `part`
// of a.ws (a key-split item, merged by flash_combine_kernel).
template <int MASK, int D, int WAVES>
__device__ __forceinline__ void flash_tile(const FlashArgs& a, const int qtile, const int head, const int b,
                                           const int k_lo, const int k_hi, const int part) {
  using C = FCfg<D, WAVES>;
  constexpr int kWaves = C::kWaves, kThreads = C::kThreads, kNB = C::kNB;
  constexpr int kTileBytes = C::kTileBytes, kVBuf = C::kVBuf, kKBuf = C::kKBuf;
  constexpr int kSmemBytes = C::kSmemBytes, kMaskBuf = C::kMaskBuf, kLoadsPerWave = C::kLoadsPerWave;
  constexpr int kMaskRing = C::kMaskRing, kCopyWaves = C::kCopyWaves;
  constexpr int kDB = C::kDB, kDS = C::kDS, kPV = C::kPV, kSlots = C::kSlots;
  constexpr bool MASKED = MASK != kMaskNone;
  constexpr int kMaskCopies = (MASK & kMaskValid ? 1 : 0) + (MASK & kMaskBias ? 1 : 0);
  constexpr bool kFull = (MASK & kMaskFull) != 0;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kSmemBytes + (MASKED ? kMaskRing * kMaskSlot : 0)];
  lds_u8* const lds = (lds_u8*)smem;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int hf = lane >> 5;   // which half of the wave
  const int col = lane & 31;  // query column within the wave's 32
  const int qw0 = (qtile * kWaves + wave) * 32;

  const bf16* qg = (const bf16*)a.q + b * a.qs[0] + head * a.qs[2];
  const bf16* kg = (const bf16*)a.k + b * a.ks[0] + head * a.ks[2];
  const bf16* vg = (const bf16*)a.v + b * a.vs[0] + head * a.vs[2];

  int kv_end = k_hi;
  if (a.kv_len != nullptr) kv_end = min(max(a.kv_len[b], 0), k_hi);
  kv_end = __builtin_amdgcn_readfirstlane(kv_end);  // uniform: scalar loop control
  const int t_begin = k_lo / kBN;                   // first key tile of the range
  const int n_tiles = (kv_end + kBN - 1) / kBN;     // one past the last key tile
  const float c = a.scale * kLog2e;

  // ---- Q (B operand of S^T = K Q^T), resident for the whole key loop.
  bf16x8 qr[kDS];
  {
    const int qi = min(qw0 + col, a.Sq - 1);
    const bf16* p = qg + (int64_t)qi * a.qs[1] + hf * 8;
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds) qr[ds] = *(const bf16x8*)(p + ds * 16);
  }

  // ---- per-lane LDS byte offsets inside one tile (half-plane 0; the
  // fragments of d 64-127 add kHalfBytes).
  // K fragment (kb, ds): key kb*32 + col, chunk 2*(ds%4) + hf of half ds/4.
  const int ksw = half_swizzle(col);
  int koff[4];
#pragma unroll
  for (int d4 = 0; d4 < 4; ++d4) koff[d4] = col * 128 + (((2 * d4 + hf) ^ ksw) * 16);
  // V transpose read (kb, j, db, e): group g = lane/16 covers columns
  // db*32 + (g%2)*16 + 0..15 of keys kb*32 + 16j + 8e + hf*4 + 0..3.
  const int i16 = lane & 15;
  const int vr = i16 >> 2, vc = i16 & 3, dh = (lane >> 4) & 1;
  // e = 0 offsets; key + 8 flips bit 0 of the swizzle, so the e = 1 offset
  // is (voff ^ 16) + 8 * 128.
  int voff[2];  // [db & 1]
#pragma unroll
  for (int db1 = 0; db1 < 2; ++db1) {
    const int key = hf * 4 + vr;
    voff[db1] = key * 128 + (((4 * db1 + 2 * dh + (vc >> 1)) ^ half_swizzle(key)) * 16) + (vc & 1) * 8;
  }
  // staging: copy i of a tile fills half-plane i / 8, keys 8*(i%8) + 0..7;
  // lane L takes key 8*(i%8) + L/8 and 16-byte column L%8
  const int srow = lane >> 3;
  const int scol = lane & 7;

  // ---- global -> LDS staging of one 64-key tile on the LDS DMA path
  // (buffer_load_dwordx4 ... lds): each wave instruction fills 8 consecutive
  // half rows (1 KiB), lane L landing at byte 16*L, so lane L fetches the
  // global chunk that the swizzle places there. kLoadsPerWave instructions
  // per copying wave per tile.
  // Tiles that lie wholly below kv_end use per-lane offsets computed once;
  // the tail tile clamps its rows to kv_end - 1.
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;
  // per-lane byte offsets of this wave's copies from the first row of a
  // tile (a tile spans 63 rows of the key stride, at most 2^24 elements:
  // well inside 32 bits); each tile's copies go through a buffer resource
  // based at its first row
  // (computed where a copying wave issues copies, so they are not live
  // in the other waves' key loop)
  struct Lanes {
    uint32_t k[kLoadsPerWave], v[kLoadsPerWave];
  };
  auto make_lanes = [&]() {
    Lanes ln;
#pragma unroll
    for (int p = 0; p < kLoadsPerWave; ++p) {
      const int i = (wave % kCopyWaves) * kLoadsPerWave + p;
      const int r = 8 * (i & 7) + srow;
      const int col_el = (i >> 3) * 64 + ((scol ^ half_swizzle(r)) * 8);
      ln.k[p] = (uint32_t)(r * (int)a.ks[1] + col_el) * 2u;
      ln.v[p] = (uint32_t)(r * (int)a.vs[1] + col_el) * 2u;
    }
    return ln;
  };
  // Byte address of this head's first k / v row and the byte distance
  // between consecutive 64-key tiles, in scalar registers: each tile's copies
  // go through one buffer resource based at the tile's first row, formed with
  // scalar adds.
  const uint64_t k_addr = uniform_u64((uint64_t)(uintptr_t)kg);
  const uint64_t v_addr = uniform_u64((uint64_t)(uintptr_t)vg);
  const uint64_t k_tile_bytes = uniform_u64((uint64_t)a.ks[1] * (2 * kBN));
  const uint64_t v_tile_bytes = uniform_u64((uint64_t)a.vs[1] * (2 * kBN));
  // this wave's copies of tile t into the LDS tile at buf_off: a whole tile
  // (every row below kv_end) issues its copies back to back with per-lane
  // offsets computed once; only the tail tile clamps its rows (one uniform
  // branch per tile and tensor)
  auto stage = [&](uint64_t addr0, uint64_t tile_bytes, const uint32_t (&lanep)[kLoadsPerWave], int64_t sstride,
                   int t, int buf_off) {
    const i32x4_rsrc rs = raw_rsrc_u64(addr0 + (uint64_t)t * tile_bytes);
    const uint32_t dst = lds_base + buf_off + (uint32_t)(wave * kLoadsPerWave) * 1024u;
    if ((t + 1) * kBN <= kv_end) {
#pragma unroll
      for (int p = 0; p < kLoadsPerWave; ++p) lds_dma16_buf(rs, lanep[p], dst + p * 1024);
    } else {
      // tail tile: rows past kv_end repeat row kv_end - 1
#pragma unroll
      for (int p = 0; p < kLoadsPerWave; ++p) {
        const int i = wave * kLoadsPerWave + p;
        const int r = 8 * (i & 7) + srow;
        const int rr = min(r, kv_end - 1 - t * kBN);
        const uint32_t voff = (uint32_t)(rr * (int)sstride + (i >> 3) * 64 + ((scol ^ half_swizzle(r)) * 8)) * 2u;
        lds_dma16_buf(rs, voff, dst + p * 1024);
      }
    }
  };
  auto stage_k = [&](const Lanes& ln, int t, int buf_off) { stage(k_addr, k_tile_bytes, ln.k, a.ks[1], t, buf_off); };
  auto stage_v = [&](const Lanes& ln, int t, int buf_off) { stage(v_addr, v_tile_bytes, ln.v, a.vs[1], t, buf_off); };

  // A per-key bias is added to a tile's scores (bias / scale for the lane's
  // keys kb*32 + g*8 + hf*4 + 0..3, from the tile's mask slot) at the top of
  // the step that takes the tile's softmax, so that scale * log2(e) * S is
  // the scaled logit plus bias * log2(e) and bias tiles stay on the fast
  // path; the QK^T accumulators of every tile start at the MFMA's inline
  // zero (a bias or zero start in registers cost 32 moves per tile). With a
  // per-(query, key) bias every tile takes the masked path anyway, and the
  // key bias is added there, next to the full bias (fewer registers).
  //
  // Key-mask tiles are classified on the device from the words staged in the
  // tile's mask slot, lane l holding word l of the tile and one ballot giving
  // the class: a tile whose 64 biases are all zero takes no bias reads or
  // adds, and a tile whose 64 validity bytes are all set takes the unmasked
  // softmax. So a key mask costs little on the tiles it leaves unmasked (a
  // padding run of -inf, or a validity hole, touches few tiles), without the
  // caller inspecting it on the host.
  const float inv_scale = 1.0f / a.scale;
  auto bias_word = [&](int j) -> float {
    return *(const VX_LDS float*)(lds + kMaskBuf + (j & (kMaskRing - 1)) * kMaskSlot + 64 + lane * 4);
  };
  auto valid_byte = [&](int j) -> uint32_t { return lds[kMaskBuf + (j & (kMaskRing - 1)) * kMaskSlot + lane]; };
  constexpr bool kKeyBias = (MASK & kMaskBias) && !kFull;     // key bias added to the scores of nonzero tiles
  constexpr bool kValidClass = (MASK & kMaskValid) && !kFull;  // (a full bias masks every tile anyway)
  auto add_key_bias = [&](int j, f32x16 (&S)[2]) {
    const lds_u8* bslot = lds + kMaskBuf + (j & (kMaskRing - 1)) * kMaskSlot + 64;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 b = *(const VX_LDS f32x4*)(bslot + (kb * 32 + g * 8 + hf * 4) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][g * 4 + e] = __builtin_fmaf(b[e], inv_scale, S[kb][g * 4 + e]);
      }
  };
  auto qk = [&](int buf_off, f32x16 (&S)[2]) {
    S[0] = f32x16{};
    S[1] = f32x16{};
    const lds_u8* kb0 = lds + buf_off;
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 kf = *(const VX_LDS bf16x8*)(kb0 + koff[ds & 3] + kb * 32 * 128 + (ds >> 2) * C::kHalfBytes);
        S[kb] = mfma32x32x16(kf, qr[ds], S[kb]);
      }
    }
  };
  auto pv = [&](int buf_off, const bf16x8 (&P)[2][2], f32x16 (&O)[kDB]) {
    const lds_u8* vb = lds + buf_off;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int db = 0; db < kDB; ++db) {
          const lds_u8* p = vb + (kb * 32 + 16 * j) * 128 + (db >> 1) * C::kHalfBytes;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + voff[db & 1]));
          const s16x4 hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + 8 * 128 + (voff[db & 1] ^ 16)));
          const bf16x8 vf = concat(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi));
          O[db] = mfma32x32x16(vf, P[kb][j], O[db]);
        }
  };
  // exp2 of the (speculative) probabilities of one tile, their bf16 packing
  // and their sum.
  auto probs = [&](const f32x16 (&S)[2], float cc, float m, bf16x8 (&P)[2][2]) -> float {
    const float mneg = -m;
    float l = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 pv8;
#pragma unroll
        for (int r = 0; r < 8; ++r) pv8[r] = (bf16)fast_exp2(__builtin_fmaf(S[kb][8 * j + r], cc, mneg));
        P[kb][j] = pv8;
        l = sum8(pv8, l);
      }
    return l;
  };

  f32x16 O[kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db) O[db] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;

  const uint8_t* vrow = (MASK & kMaskValid) ? a.key_valid + (int64_t)b * a.key_mask_stride : nullptr;
  // this lane's query row of the full bias (row of a clamped query past Sq)
  const float* frow = kFull ? a.full_bias + b * a.fbs[0] + head * a.fbs[1] +
                                  (int64_t)min(qw0 + col, a.Sq - 1) * a.fbs[2]
                            : nullptr;
  const float* brow = (MASK & kMaskBias) ? a.key_bias + (int64_t)b * a.key_mask_stride : nullptr;
  // Wave 0 stages tile j's mask (64 validity bytes: lanes 0-3; 64 biases:
  // lanes 0-15) into mask slot j % kMaskRing. Mask rows hold whole 64-key
  // tiles.
  // (buffer form from the batch item's mask row in scalar registers, so the
  // per-lane part of the source is a small constant offset)
  const uint64_t vrow_addr = uniform_u64((uint64_t)(uintptr_t)vrow);
  const uint64_t brow_addr = uniform_u64((uint64_t)(uintptr_t)brow);
  auto stage_mask = [&](int j) {
    if (!MASKED || wave != 0) return;
    const uint32_t slot = lds_base + kMaskBuf + (j & (kMaskRing - 1)) * kMaskSlot;
    if (MASK & kMaskValid) {
      if (lane < 4) lds_dma16_buf(raw_rsrc_u64(vrow_addr + (uint64_t)j * kBN), lane * 16, slot);
    }
    if (MASK & kMaskBias) {
      if (lane < 16) lds_dma16_buf(raw_rsrc_u64(brow_addr + (uint64_t)j * kBN * 4), lane * 16, slot + 64);
    }
  };
  // At the top of iteration t: the tiles it reads (K_{t+1}, V_{t-1}) were
  // issued kNB - 1 iterations earlier; the copies of the last kNB - 2
  // iterations may still be in flight.
  auto wait_prev = [&]() {
    if (MASKED && wave == 0)
      wait_vmem<(kNB - 2) * (2 * kLoadsPerWave + kMaskCopies)>();
    else
      wait_vmem<(kNB - 2) * 2 * kLoadsPerWave>();
  };

  if (n_tiles > t_begin) {
    // Tile j of K lives in K buffer j % kNB and tile j of V in V buffer
    // j % kNB; V buffer kNB-1 stands in for "V_{-1}" (zeros, paired with P = 0
    // in iteration 0). Iteration t issues K_{t+kNB}, the mask of tile
    // t+kNB+1 and V_{t+kNB-2}, into the buffers that the previous iteration
    // finished reading; the prologue issues the first mask and then the same
    // groups for t = -kNB .. -1, so that every wait below counts whole
    // groups (the first mask is older than all of them).
    if (wave < kCopyWaves) {
      const Lanes ln = make_lanes();
      stage_mask(t_begin);  // (masks run one tile ahead of K: the first one on its own)
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        stage_k(ln, min(t_begin + j, n_tiles - 1), kKBuf + j * kTileBytes);
        stage_mask(min(t_begin + j + 1, n_tiles - 1));
        if (j >= 2) stage_v(ln, min(t_begin + j - 2, n_tiles - 1), kVBuf + (j - 2) * kTileBytes);
      }
    }
#pragma unroll
    for (int p = 0; p < kTileBytes / (kThreads * 16); ++p)
      *(VX_LDS u32x4*)(lds + kVBuf + (kNB - 1) * kTileBytes + (p * kThreads + threadIdx.x) * 16) = u32x4{0, 0, 0, 0};
    // K_0 has landed (with two tiles per ring, K_1 may still be in flight;
    // with more, K_1 has landed too)
    if (kNB == 2) {
      if (MASKED && wave == 0)
        wait_vmem<kLoadsPerWave + kMaskCopies>();
      else
        wait_vmem<kLoadsPerWave>();
    } else {
      wait_prev();
    }
    __syncthreads();
    f32x16 S[2];
    qk(kKBuf, S);
    bf16x8 Pp[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j) Pp[kb][j] = bf16x8{};

    int kb_cur = 1;         // K buffer holding K_{t+1}  (= (t+1) % kNB)
    int vb_prev = kNB - 1;  // V buffer holding V_{t-1}  (= (t+kNB-1) % kNB)
    // the current tile has an invalid key (each step classifies the next one)
    bool invalid_cur = kValidClass && __builtin_amdgcn_ballot_w64(valid_byte(t_begin) == 0) != 0;
    // the current tile has a nonzero key bias (each step classifies the next one)
    bool bias_nz_cur = kKeyBias && __builtin_amdgcn_ballot_w64(bias_word(t_begin) != 0.f) != 0;
    // One key tile: consumes S (scores of tile t) and Pp (probabilities of
    // tile t-1), produces Sn (scores of tile t+1) and P (probabilities of
    // tile t). The loop below calls it twice per trip with the two register
    // sets swapped, so no copies are needed between tiles.
    // COPY (a compile-time tag): this wave issues tile copies. The 8-wave
    // workgroups run two copies of the loop, one for the copying waves and
    // one for the others, so that neither carries the other's branches.
    auto step = [&](auto copy_tag, const Lanes& ln, const int t, f32x16 (&S)[2], f32x16 (&Sn)[2],
                    const bf16x8 (&Pp)[2][2], bf16x8 (&P)[2][2]) __attribute__((always_inline)) {
      constexpr bool COPY = decltype(copy_tag)::value;
      // K_{t+1} and V_{t-1} have landed once wait_prev returns; the barrier
      // then publishes them, and it also frees K buffer t % kNB (K_t, read by
      // QK(t) last iteration) and V buffer (t+kNB-2) % kNB (V_{t-2}) for this
      // iteration's copies.
      wait_prev();
      __syncthreads();
      // the class words of tile t+1's validity and bias (its mask slot has
      // landed: masks run a tile ahead of K), read first so that their
      // latency is covered by the work below; both classes are taken at the
      // end of this step, for the next one
      float bias_next = 0.f;
      uint32_t valid_next = 1;
      if (kKeyBias) bias_next = bias_word(min(t + 1, n_tiles - 1));
      if (kValidClass) valid_next = valid_byte(t + 1);
      // tile t's key bias, into its scores (a tile classified nonzero)
      if (kKeyBias && bias_nz_cur) add_key_bias(t, S);
      const int kb_next = kb_cur == 0 ? kNB - 1 : kb_cur - 1;     // t % kNB
      const int vb_next = vb_prev == 0 ? kNB - 1 : vb_prev - 1;  // (t+kNB-2) % kNB

      // ---- key masks. Tiles that hold a masked key (the tail tile, a
      // key_valid hole) take the scores to log2 units here, masked keys ->
      // -inf, and use cc = 1 below; fully valid tiles (and key bias tiles,
      // whose bias is in the scores already) keep the fused scale in the exp
      // argument.
      const int key0 = t * kBN;
      const lds_u8* mslot = lds + kMaskBuf + (t & (kMaskRing - 1)) * kMaskSlot;  // tile t's mask
      bool slow = key0 + kBN > kv_end;
      if (kValidClass) slow = slow || invalid_cur;  // tile t has an invalid key (classified last step)
      if (MASK & kMaskFull) slow = true;
      // this iteration's copies: K_{t+kNB}, the mask of tile t+kNB+1 and V_{t+kNB-2}
      if (COPY) {
        stage_k(ln, min(t + kNB, n_tiles - 1), kKBuf + kb_next * kTileBytes);
        stage_mask(min(t + kNB + 1, n_tiles - 1));
        stage_v(ln, min(t + kNB - 2, n_tiles - 1), kVBuf + vb_next * kTileBytes);
      }
      float cc = c;
      if (slow) {
        cc = 1.0f;
        // this lane's validity bytes: keys kb*32 + g*8 + hf*4 + 0..3
        uint32_t vbits[2][4];
        if (MASK & kMaskValid) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int g = 0; g < 4; ++g) vbits[kb][g] = *(const VX_LDS uint32_t*)(mslot + kb * 32 + g * 8 + hf * 4);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int kbase = key0 + kb * 32 + g * 8 + hf * 4;
            f32x4 bias = {0.f, 0.f, 0.f, 0.f};
            if (kFull) bias += *(const f32x4*)(frow + kbase) * kLog2e;
            if (kFull && (MASK & kMaskBias))
              bias += *(const VX_LDS f32x4*)(mslot + 64 + (kb * 32 + g * 8 + hf * 4) * 4) * kLog2e;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              bool ok = kbase + e < kv_end;
              if (MASK & kMaskValid) ok = ok && ((vbits[kb][g] >> (8 * e)) & 0xffu) != 0;
              const float sv = __builtin_fmaf(S[kb][g * 4 + e], c, bias[e]);
              S[kb][g * 4 + e] = ok ? sv : -__builtin_inff();
            }
          }
        }
      }

      // ---- the MFMA block: 32 slots, slot s issues one MFMA (s < 16:
      // PV(t-1) into O, s >= 16: QK^T(t+1) into Sn) and the LDS read of the
      // fragment three slots ahead. The softmax of tile t (speculative
      // against the current max) runs as a separate VALU block: with two
      // waves per SIMD, one wave's MFMA block overlaps the other wave's VALU
      // block, which measured 1.5 % faster at L=32760 than interleaving one
      // score's exp into every slot (and no slower with 4 waves). In 8-wave
      // workgroups the VALU block follows the MFMAs, in 4-wave workgroups it
      // precedes them.
      float l_tile = 0.f;
      {
        const lds_u8* kb0 = lds + kKBuf + kb_cur * kTileBytes;
        const lds_u8* vb0 = lds + kVBuf + vb_prev * kTileBytes;
        // slot s < kPV: PV fragment (kb, j, db) with s = (kb * 2 + j) * kDB + db;
        // slot s >= kPV: QK^T fragment (ds, kb) with s - kPV = 2 * ds + kb.
        auto frag = [&](int s) -> bf16x8 {
          if (s < kPV) {
            const int db = s % kDB, j = (s / kDB) & 1, kb = s / (2 * kDB);
            const lds_u8* p = vb0 + (kb * 32 + 16 * j) * 128 + (db >> 1) * C::kHalfBytes;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + voff[db & 1]));
            const s16x4 hi =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + 8 * 128 + (voff[db & 1] ^ 16)));
            return concat(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi));
          }
          const int ds = (s - kPV) >> 1, kb = (s - kPV) & 1;
          return *(const VX_LDS bf16x8*)(kb0 + koff[ds & 3] + kb * 32 * 128 + (ds >> 2) * C::kHalfBytes);
        };
        const float mneg = -m_run;
        const bf16x2 one2 = {(bf16)1.0f, (bf16)1.0f};
        // Wave priority 1 while in the slots: with 8 waves for the waves that
        // issue no copies (they start their slots first; the copying waves
        // fill the gaps they leave: +0.7 %), with 4 waves (two workgroups per
        // CU) for every wave, ahead of the other workgroup's wave while that
        // one copies, waits or starts (+2-4 % at 512 keys).
        constexpr bool kAllPrio = WAVES == 4;
        if (kAllPrio || !COPY) __builtin_amdgcn_s_setprio(1);
        bf16x8 fr[kSlots];
        float pf[32];
        bf16x2 pk[16];
        fr[0] = frag(0);
        fr[1] = frag(1);
        fr[2] = frag(2);
        // softmax block: 4 groups of 8 scores (8 FMAs, 8 exps, 4 packs each),
        // then the 16 pair sums of the tile
        auto softmax_block = [&]() {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int i = 0; i < 8; ++i) pf[8 * g + i] = __builtin_fmaf(S[g >> 1][8 * (g & 1) + i], cc, mneg);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 8; ++i) pf[8 * g + i] = fast_exp2(pf[8 * g + i]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i) pk[4 * g + i] = bf16x2{(bf16)pf[8 * g + 2 * i], (bf16)pf[8 * g + 2 * i + 1]};
            __builtin_amdgcn_sched_barrier(0);
          }
#pragma unroll
          for (int i = 0; i < 16; ++i) l_tile = __builtin_amdgcn_fdot2_f32_bf16(pk[i], one2, l_tile, false);
          __builtin_amdgcn_sched_barrier(0);
        };
        if (WAVES == 4 || COPY) softmax_block();
        // read by the QK^T slots (16 and on)
        Sn[0] = f32x16{};
        Sn[1] = f32x16{};
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
          if (s + 3 < kSlots) fr[s + 3] = frag(s + 3);
          if (s < kPV) {
            const int db = s % kDB, j = (s / kDB) & 1, kb = s / (2 * kDB);
            O[db] = mfma32x32x16(fr[s], Pp[kb][j], O[db]);
          } else {
            const int ds = (s - kPV) >> 1, kb = (s - kPV) & 1;
            Sn[kb] = mfma32x32x16(fr[s], qr[ds], Sn[kb]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (kAllPrio || !COPY) __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        if (WAVES == 8 && !COPY) softmax_block();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int q = kb * 8 + j * 4;
            P[kb][j] = __builtin_shufflevector(__builtin_shufflevector(pk[q], pk[q + 1], 0, 1, 2, 3),
                                               __builtin_shufflevector(pk[q + 2], pk[q + 3], 0, 1, 2, 3),
                                               0, 1, 2, 3, 4, 5, 6, 7);
          }
      }

      // ---- rare: a probability may exceed 2^kRescaleSlack (the lane's tile
      // sum is above kSumLimit, inf or NaN; the first tile always lands here
      // because m_run starts at kNegBig) -> raise the reference point to the
      // tile max, rescale O and l, recompute this tile's probabilities.
      if (__builtin_amdgcn_ballot_w64(l_tile > kSumLimit || is_nan_bits(l_tile)) != 0) {
        float mxc = -__builtin_inff();
#pragma unroll
        for (int e = 0; e < 16; ++e) mxc = __builtin_fmaxf(__builtin_fmaxf(mxc, S[0][e]), S[1][e]);
        const float mn = fmaxf(m_run, halves_max(mxc) * cc);
        const float alpha = fast_exp2(m_run - mn);
        m_run = mn;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < kDB; ++db) O[db] *= alpha;
        l_tile = probs(S, cc, m_run, P);
      }
      l_run += l_tile;
      kb_cur = kb_cur == kNB - 1 ? 0 : kb_cur + 1;
      vb_prev = vb_prev == kNB - 1 ? 0 : vb_prev + 1;
      if (kValidClass) invalid_cur = __builtin_amdgcn_ballot_w64(valid_next == 0) != 0;
      if (kKeyBias) bias_nz_cur = __builtin_amdgcn_ballot_w64(bias_next != 0.f) != 0;
    };

    f32x16 S2[2];
    bf16x8 P2[2][2];
    auto key_loop = [&](auto copy_tag) __attribute__((always_inline)) {
      Lanes ln{};
      if constexpr (decltype(copy_tag)::value) ln = make_lanes();
      int t = t_begin;
      for (; t + 1 < n_tiles; t += 2) {
        step(copy_tag, ln, t, S, S2, Pp, P2);
        step(copy_tag, ln, t + 1, S2, S, P2, Pp);
      }
      if (t < n_tiles) {
        step(copy_tag, ln, t, S, S2, Pp, P2);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 2; ++j) Pp[kb][j] = P2[kb][j];
      }
    };
    if (kCopyWaves == kWaves || wave < kCopyWaves)
      key_loop(std::integral_constant<bool, true>{});
    else
      key_loop(std::integral_constant<bool, kCopyWaves == kWaves>{});
    // ---- PV of the last tile (V_{n-1} sits in V buffer vb_prev now).
    wait_vmem<0>();
    __syncthreads();
    pv(kVBuf + vb_prev * kTileBytes, Pp, O);
  }

  // ---- key-split item: the unnormalised accumulators, the reference point
  // and this lane's part of the row sum go to partial slot `part` (lane
  // order, one 1 KiB wave store per 16 bytes of each lane).
  if (part >= 0) {
    f32x4* slot = (f32x4*)(a.ws + (int64_t)part * flash_part_floats(kWaves, D));
    f32x4* wo = slot + (int64_t)wave * (kDB * 4) * 64 + lane;
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4)
        wo[(db * 4 + k4) * 64] = f32x4{O[db][4 * k4], O[db][4 * k4 + 1], O[db][4 * k4 + 2], O[db][4 * k4 + 3]};
    float* ml = (float*)(slot + (int64_t)kWaves * kDB * 4 * 64) + 2 * (wave * 64 + lane);
    *(float2*)ml = float2{m_run, l_run};
    return;
  }

  // ---- epilogue: normalise, pack to 16-byte chunks of 8 consecutive d,
  // regroup into whole lines and store.
  const float lt = halves_sum(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  // (the output address is formed here, so nothing of it is live in the key loop)
  store_out_lines<kDB>(O, inv, (bf16*)a.o + (b * a.os[0] + head * a.os[2]), qw0, a.Sq, a.os[1], lane);
}

template <int MASK, int D, int WAVES>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_fwd_kernel(const FlashArgs a) {
  flash_tile<MASK, D, WAVES>(a, blockIdx.x, blockIdx.y, blockIdx.z, 0, a.Sk, -1);
}

// Key-split launch: items (query tile fastest, then head, then batch item)
// below n_full run whole; each of the last a.split_items items runs as two
// workgroups, over keys [0, k_mid) and [k_mid, Sk), writing partials.
template <int MASK, int D, int WAVES>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_fwd_split_kernel(const FlashArgs a, int n_full, int n_qt) {
  const int w = blockIdx.x;
  int item = w, k_lo = 0, k_hi = a.Sk, part = -1;
  if (w >= n_full) {
    part = w - n_full;
    item = n_full + (part >> 1);
    if (part & 1)
      k_lo = a.k_mid;
    else
      k_hi = a.k_mid;
  }
  const int qt = item % n_qt, bh = item / n_qt;
  flash_tile<MASK, D, WAVES>(a, qt, bh % a.H, bh / a.H, k_lo, k_hi, part);
}

// Merges the two key halves of each split item: with M the larger reference
// point, O = (O0 2^(m0-M) + O1 2^(m1-M)) / (l0 2^(m0-M) + l1 2^(m1-M)),
// packed and stored as the main kernel's epilogue does (same lane layout).
template <int D, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void flash_combine_kernel(const FlashArgs a, int n_full, int n_qt) {
  constexpr int kDB = D / 32;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hf = lane >> 5, col = lane & 31;
  const int item = n_full + blockIdx.x;
  const int qt = item % n_qt, bh = item / n_qt, head = bh % a.H, b = bh / a.H;
  const f32x4* s0 = (const f32x4*)(a.ws + (int64_t)(2 * blockIdx.x) * flash_part_floats(WAVES, D));
  const f32x4* s1 = (const f32x4*)(a.ws + (int64_t)(2 * blockIdx.x + 1) * flash_part_floats(WAVES, D));
  const int ml_idx = 2 * (wave * 64 + lane);
  const float2 ml0 = *(const float2*)((const float*)(s0 + (int64_t)WAVES * kDB * 4 * 64) + ml_idx);
  const float2 ml1 = *(const float2*)((const float*)(s1 + (int64_t)WAVES * kDB * 4 * 64) + ml_idx);
  const float M = fmaxf(ml0.x, ml1.x);
  const float a0 = fast_exp2(ml0.x - M), a1 = fast_exp2(ml1.x - M);
  const float lt = halves_sum(ml0.y * a0 + ml1.y * a1);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  f32x16 O[kDB];
  const int64_t base = (int64_t)wave * (kDB * 4) * 64 + lane;
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const f32x4 x0 = s0[base + (db * 4 + k4) * 64], x1 = s1[base + (db * 4 + k4) * 64];
#pragma unroll
      for (int e = 0; e < 4; ++e) O[db][4 * k4 + e] = x0[e] * a0 + x1[e] * a1;
    }
  store_out_lines<kDB>(O, inv, (bf16*)a.o + b * a.os[0] + head * a.os[2], (qt * WAVES + wave) * 32, a.Sq, a.os[1],
                       lane);
}

// ---- persistent kernel for short key sequences (key masks: kv_len only).
//
// One 8-wave workgroup per CU. Each workgroup takes a contiguous range of
// (256-query tile, head, batch item) items, the ranges cut so that every
// workgroup gets about the same number of key tiles (each item counted with
// one tile more for its start and end), and runs the key tiles of its items
// as one stream u = 0, 1, ...: step u takes the softmax of stream tile u,
// PV of tile u-1 and QK^T of tile u+1 in its MFMA slots, and copies K_{u+3}
// and V_{u+1}, whichever items these tiles belong to. So the next item's
// first tiles are copied while the current item ends; the QK^T slots of an
// item's last step score the next item's first tile (its q tile was copied
// into LDS at the item's first step and is read into registers at the top
// of that last step); and the PV slots of an item's first step finish the
// previous item, whose output rows are stored at the end of that step. The
// 256-query items copy half the K/V bytes per query of 128-query
// workgroups, and the stream takes each item's pipeline fill and drain
// (q load, first copies, last PV and stores) off the critical path.
// Workgroup g runs on XCD g % 8 (round-robin dispatch), and the XCDs take
// contiguous eighths of the items, so that each XCD's L2 holds the K/V of
// few heads. Items of a batch item with kv_len 0 get zero rows.
template <int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_stream_kernel(const FlashArgs a) {
  using C = FCfg<D, 8>;
  constexpr int kWaves = 8, kThreads = 512;
  constexpr int kTileBytes = C::kTileBytes;
  constexpr int kLoadsPerWave = C::kLoadsPerWave, kCopyWaves = C::kCopyWaves;
  constexpr int kDB = C::kDB, kDS = C::kDS, kPV = C::kPV, kSlots = C::kSlots;
  // LDS: two V tiles (V_u is copied in step u and read in step u+1), three
  // K tiles (K_{u+3} copied in step u, read in step u+2), the next item's q
  // tile (four 64-row tiles in the K layout) and the table of the
  // workgroup's items (kTabMax entries of 16 bytes: batch item, head, query
  // tile, keys; the launcher keeps every workgroup within it)
  constexpr int kKNB = 3;
  constexpr int kVBuf = 0, kKBuf = 2 * kTileBytes, kQBuf = 5 * kTileBytes, kTab = 9 * kTileBytes;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kTab + kStreamTabMax * 16];
  lds_u8* const lds = (lds_u8*)smem;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hf = lane >> 5, col = lane & 31;
  const int n_qt = (a.Sq + 255) / 256;
  const int per_b = a.H * n_qt;  // items per batch item
  auto uni = [](int x) { return __builtin_amdgcn_readfirstlane(x); };
  auto kv_end_of = [&](int b) __attribute__((always_inline)) -> int {
    int kv = a.Sk;
    if (a.kv_len != nullptr) kv = min(max(a.kv_len[b], 0), a.Sk);
    return uni(kv);
  };
  auto tiles_of = [](int kv) { return (kv + kBN - 1) / kBN; };

  // ---- this workgroup's items [i_lo, i_hi): item j of batch item b starts
  // at work P_b + j * (n_b + kItemTiles), P_b the work of the batch items
  // before b. An item's start and end (its q tile copy, the first tile's
  // max, the output stores) cost about kItemTiles key tiles of the stream:
  // with 1 instead of 3 the workgroups holding the short items of a batch
  // with mixed kv_len finished late (same box: 32760 x 512 with kv_len
  // 432 / 148 0.679 -> 0.634 ms, 32760 x 256 with 200 / 60 0.633 -> 0.540
  // ms, 16384 x 1024 with 1000 / 700 / 300 / 30 1.394 -> 0.968 ms; equal
  // items unchanged).
  constexpr int kItemTiles = 3;
  int64_t W = 0;
  for (int b = 0; b < a.B; ++b) W += (int64_t)per_b * (tiles_of(kv_end_of(b)) + kItemTiles);
  const int G = gridDim.x;
  const int chunk_id = (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8;
  auto first_item_at = [&](int64_t x) __attribute__((always_inline)) -> int {  // first item starting at or after work x
    int64_t P = 0;
    for (int b = 0; b < a.B; ++b) {
      const int w = tiles_of(kv_end_of(b)) + kItemTiles;
      const int64_t end = P + (int64_t)per_b * w;
      if (x < end) return b * per_b + (int)((x - P + w - 1) / w);
      P = end;
    }
    return a.B * per_b;
  };
  const int i_lo = uni(first_item_at(W * chunk_id / G));
  const int i_hi = uni(first_item_at(W * (chunk_id + 1) / G));

  // stream length; items of batch items with no keys get zero rows
  int U = 0;
  for (int b = i_lo / per_b; b < a.B && b * per_b < i_hi; ++b) {
    const int lo = max(i_lo, b * per_b), hi = min(i_hi, (b + 1) * per_b);
    const int n = tiles_of(kv_end_of(b));
    U += (hi - lo) * n;
    if (n == 0) {
      for (int i = lo; i < hi; ++i) {
        const int r = i - b * per_b, h = r / n_qt, qi = (r % n_qt * kWaves + wave) * 32 + col;
        if (qi < a.Sq) {
          bf16* orow = (bf16*)a.o + (b * a.os[0] + h * a.os[2]) + (int64_t)qi * a.os[1];
#pragma unroll
          for (int db = 0; db < kDB; ++db)
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) *(u32x4*)(orow + db * 32 + (2 * pr + hf) * 8) = u32x4{0, 0, 0, 0};
        }
      }
    }
  }
  U = uni(U);
  if (U == 0) return;

  // ---- the table of this workgroup's items with keys (built by all
  // threads; entry e of the items in [i_lo, i_hi) minus those of batch items
  // without keys before it)
  int n_items = 0;
  for (int b = i_lo / per_b; b < a.B && b * per_b < i_hi; ++b)
    if (kv_end_of(b) > 0) n_items += min(i_hi, (b + 1) * per_b) - max(i_lo, b * per_b);
  n_items = uni(n_items);
  for (int e = threadIdx.x; e < i_hi - i_lo; e += kThreads) {
    const int i = i_lo + e, b = i / per_b;
    const int kv = a.kv_len != nullptr ? min(max(a.kv_len[b], 0), a.Sk) : a.Sk;
    if (kv == 0) continue;
    int skip = 0;
    for (int bb = i_lo / per_b; bb < b; ++bb) {
      const int kvb = a.kv_len != nullptr ? min(max(a.kv_len[bb], 0), a.Sk) : a.Sk;
      if (kvb == 0) skip += min(i_hi, (bb + 1) * per_b) - max(i_lo, bb * per_b);
    }
    const int r = i - b * per_b, h = r / n_qt;
    if (e - skip < kStreamTabMax)  // (always: the launcher sizes the grid so)
      *(VX_LDS i32x4*)(lds + kTab + (e - skip) * 16) = i32x4{b, h, r - h * n_qt, kv};
  }
  __syncthreads();
  struct Item {
    int b, h, qt, kv;
  };
  auto entry = [&](int e) __attribute__((always_inline)) -> Item {
    const i32x4 v = *(const VX_LDS i32x4*)(lds + kTab + e * 16);
    return Item{uni(v[0]), uni(v[1]), uni(v[2]), uni(v[3])};
  };

  // ---- LDS offsets (the layout of flash_tile: half-planes of 64 rows x
  // 128 bytes, 16-byte chunks XOR-swizzled per row)
  // K fragment (kb, ds): key kb*32 + col, chunk 2*(ds%4) + hf of half ds/4,
  // at koff0 ^ ((ds % 4) << 5) (2*(ds%4) + hf = 2*(ds%4) ^ hf).
  const int koff0 = col * 128 + ((hf ^ half_swizzle(col)) * 16);
  auto kofs = [&](int d4) { return koff0 ^ (d4 << 5); };
  const int i16 = lane & 15;
  const int vr = i16 >> 2, vc4 = i16 & 3, dh = (lane >> 4) & 1;
  int voff[2];
#pragma unroll
  for (int db1 = 0; db1 < 2; ++db1) {
    const int key = hf * 4 + vr;
    voff[db1] = key * 128 + (((4 * db1 + 2 * dh + (vc4 >> 1)) ^ half_swizzle(key)) * 16) + (vc4 & 1) * 8;
  }
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;
  const uint64_t q_addr = uniform_u64((uint64_t)(uintptr_t)a.q);
  const uint64_t k_addr = uniform_u64((uint64_t)(uintptr_t)a.k);
  const uint64_t v_addr = uniform_u64((uint64_t)(uintptr_t)a.v);
  const uint64_t k_tile_bytes = uniform_u64((uint64_t)a.ks[1] * (2 * kBN));
  const uint64_t v_tile_bytes = uniform_u64((uint64_t)a.vs[1] * (2 * kBN));
  // this wave's copies of 64 rows from byte address `addr` into the LDS tile
  // at buf_off; rows from rows_left on repeat row rows_left - 1 (>= 0)
  // (the per-lane offsets of whole tiles are loop-invariant, held in
  // registers: forming them at each call, to keep registers free, cost 3 %
  // at 32760 x 512 keys)
  auto stage_clamped = [&](uint64_t addr, int64_t stride, int rows_left, int buf_off) __attribute__((always_inline)) {
    const i32x4_rsrc rs = raw_rsrc_u64(addr);
    const uint32_t dst = lds_base + buf_off + (uint32_t)(wave * kLoadsPerWave) * 1024u;
    const int sr = lane >> 3, sc = lane & 7;
    if (rows_left >= kBN) {
      // row r = 8*(i%8) + sr: its swizzle depends on sr and on bit 0 of i,
      // the rest of the offset is uniform
      const uint32_t lane0 = (uint32_t)(sr * (int)stride + ((sc ^ half_swizzle(sr)) * 8)) * 2u;
      const uint32_t lane1 = (uint32_t)(sr * (int)stride + ((sc ^ half_swizzle(sr + 8)) * 8)) * 2u;
#pragma unroll
      for (int p = 0; p < kLoadsPerWave; ++p) {
        const int i = wave * kLoadsPerWave + p;
        const uint32_t row0 = (uint32_t)(8 * (i & 7) * (int)stride + (i >> 3) * 64) * 2u;
        lds_dma16_buf(rs, ((i & 1) ? lane1 : lane0) + row0, dst + p * 1024);
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < kLoadsPerWave; ++p) {
      const int i = wave * kLoadsPerWave + p;
      const int r = 8 * (i & 7) + sr;
      const int rr = min(r, rows_left - 1);
      const uint32_t off = (uint32_t)(rr * (int)stride + (i >> 3) * 64 + ((sc ^ half_swizzle(r)) * 8)) * 2u;
      lds_dma16_buf(rs, off, dst + p * 1024);
    }
  };
  // q rows of table entry e (4 x 64 rows; rows past Sq repeat row Sq - 1)
  auto stage_q = [&](int e) __attribute__((always_inline)) {
    const Item it = entry(e);
    const uint64_t head = q_addr + (uint64_t)((int64_t)it.b * a.qs[0] + (int64_t)it.h * a.qs[2]) * 2u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r0 = min(it.qt * 256 + 64 * j, a.Sq - 1);
      stage_clamped(head + (uint64_t)((int64_t)r0 * a.qs[1]) * 2u, a.qs[1], a.Sq - r0, kQBuf + j * kTileBytes);
    }
  };
  // this wave's 32 q rows from the q buffer (the B operand of QK^T)
  auto load_q = [&](bf16x8 (&qr)[kDS]) __attribute__((always_inline)) {
    const lds_u8* qb = lds + kQBuf + (wave >> 1) * kTileBytes + (wave & 1) * 32 * 128;
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds)
      qr[ds] = *(const VX_LDS bf16x8*)(qb + kofs(ds & 3) + (ds >> 2) * C::kHalfBytes);
  };

  // ---- copy cursors (wave-uniform): byte address of the tile's first row,
  // its rows below kv_end, the tiles left in its item, its table entry.
  // After the stream's last tile a cursor stays there (that tile is copied
  // again).
  struct CopyCur {
    uint64_t addr;
    int rows, left, e;
  };
  auto open_copy = [&](CopyCur& c, int e, uint64_t base, const int64_t (&s)[3]) __attribute__((always_inline)) {
    const Item it = entry(e);
    c.e = e;
    c.rows = it.kv;
    c.left = tiles_of(it.kv);
    c.addr = uniform_u64(base + (uint64_t)((int64_t)it.b * s[0] + (int64_t)it.h * s[2]) * 2u);
  };
  auto advance_copy = [&](CopyCur& c, uint64_t base, const int64_t (&s)[3], uint64_t tile_bytes) __attribute__((always_inline)) {
    if (c.left > 1) {
      --c.left;
      c.rows -= kBN;
      c.addr += tile_bytes;
      return;
    }
    if (c.e + 1 < n_items) open_copy(c, c.e + 1, base, s);
  };

  // ---- the scored tile (wave-uniform): table entry, tile in it, its tiles
  // and keys
  int c_e = 0;
  int c_kv = entry(0).kv;
  int c_n = tiles_of(c_kv), c_t = 0;
  bool has_prev = false;

  const float c = a.scale * kLog2e;
  f32x16 O[kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db) O[db] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;

  // output rows of table entry e, normalised by the row sum l (one 32-wide
  // d block at a time: few registers, as it runs inside the key loop).
  // Every wave issues exactly 2 * kDB store instructions, which the copying
  // waves' waits count, so a wave never skips one. Lanes past Sq hold row
  // Sq-1's query (the q copies repeat that row) but must not store it: their
  // probabilities may round differently from the owner's (the rare rescale
  // is taken per wave). The stores go through a buffer resource that ends at
  // the item's last row below Sq, and those lanes' offsets lie past its end,
  // where the hardware drops the write (the instruction still counts).
  const uint64_t o_addr = uniform_u64((uint64_t)(uintptr_t)a.o);
  auto epilogue = [&](int e, float l) __attribute__((always_inline)) {
    const float lt = halves_sum(l);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    const Item it = entry(e);
    const int r0 = it.qt * 256;                   // the item's first query row
    const int rows = uni(min(256, a.Sq - r0));    // its rows below Sq
    // (offsets below 2^31: the plan keeps the output's row stride <= 2^22 elements)
    const uint64_t base =
        o_addr + (uint64_t)((int64_t)it.b * a.os[0] + (int64_t)it.h * a.os[2] + (int64_t)r0 * a.os[1]) * 2u;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(uintptr_t)base, (short)0, (int)(((int64_t)(rows - 1) * a.os[1] + D) * 2), 0x00020000);
    // whole 128-byte lines (line_chunks): lane l stores rows (l & 7) + 8 i of
    // its wave; one 64-wide d pair at a time (few registers)
    uint32_t off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = wave * 32 + (lane & 7) + 8 * i;
      off[i] = q < rows ? (uint32_t)(q * (int)a.os[1]) * 2u : 0x80000000u;
    }
#pragma unroll
    for (int p = 0; p < kDB / 2; ++p) {
      u32x4 chunk[2][2];
      const f32x16 Ob[2] = {O[2 * p], O[2 * p + 1]};
      pack_out_rows<2>(Ob, inv, chunk);
      u32x4 out[4];
      line_chunks(chunk, out);
      const uint32_t cofs = line_chunk_offset(lane, p);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, out[i]), rs, off[i] + cofs, 0, 0);
    }
  };
  auto probs = [&](const f32x16 (&S)[2], float cc_, float m, bf16x8 (&P)[2][2]) __attribute__((always_inline)) -> float {
    const float mneg = -m;
    float l = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 pv8;
#pragma unroll
        for (int r = 0; r < 8; ++r) pv8[r] = (bf16)fast_exp2(__builtin_fmaf(S[kb][8 * j + r], cc_, mneg));
        P[kb][j] = pv8;
        l = sum8(pv8, l);
      }
    return l;
  };

  // ---- prologue: q of the first item, K_0..K_2; V buffer 1 is "V_{-1}"
  // (zeros, paired with P = 0 in step 0)
  CopyCur kc{}, vc{};
  bf16x8 qr[kDS];
  if (wave < kCopyWaves) {
    open_copy(kc, 0, k_addr, a.ks);
    open_copy(vc, 0, v_addr, a.vs);
    stage_q(0);
#pragma unroll
    for (int j = 0; j < kKNB; ++j) {
      stage_clamped(kc.addr, a.ks[1], kc.rows, kKBuf + j * kTileBytes);
      advance_copy(kc, k_addr, a.ks, k_tile_bytes);
    }
  }
#pragma unroll
  for (int p = 0; p < kTileBytes / (kThreads * 16); ++p)
    *(VX_LDS u32x4*)(lds + kVBuf + kTileBytes + (p * kThreads + threadIdx.x) * 16) = u32x4{0, 0, 0, 0};
  // Step u copies V_u, then K_{u+3}: at its top, V_{u-1} (the previous
  // step's first copies) and K_{u+1} have landed; the previous step's K copy
  // may still be in flight, and so may the output stores issued after it
  // (`stored`: the previous step ended an item). Only the copying waves
  // wait; the barrier after the wait publishes their copies to all waves.
  bool stored = false;
  auto wait_prev = [&]() __attribute__((always_inline)) {
    if (wave < kCopyWaves) {
      if (stored)
        wait_vmem<kLoadsPerWave + 2 * kDB>();
      else
        wait_vmem<kLoadsPerWave>();
    }
  };
  wait_prev();
  __syncthreads();
  // q of the first item and the scores of its first tile, formed at the top
  // of each wave kind's loop (below): formed before the branch into the two
  // loops, q was spilled across it
  f32x16 S[2];
  bf16x8 Pp[2][2];
  auto first_scores = [&]() __attribute__((always_inline)) {
    load_q(qr);
    S[0] = f32x16{};
    S[1] = f32x16{};
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 kf =
            *(const VX_LDS bf16x8*)(lds + kKBuf + kofs(ds & 3) + kb * 32 * 128 + (ds >> 2) * C::kHalfBytes);
        S[kb] = mfma32x32x16(kf, qr[ds], S[kb]);
      }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j) Pp[kb][j] = bf16x8{};
  };

  int kb_cur = 1;   // K buffer holding K_{u+1}
  int vb_prev = 1;  // V buffer holding V_{u-1}
  // Stream step u (flash_tile's step; the item changes happen between
  // steps, below): consumes S (scores of tile u) and Pp (probabilities of
  // tile u-1), produces Sn (scores of tile u+1) and P (probabilities of tile
  // u); returns the row sum of P (this lane's part).
  auto step = [&](auto copy_tag, const int u, f32x16 (&S)[2], f32x16 (&Sn)[2],
                  const bf16x8 (&Pp)[2][2], bf16x8 (&P)[2][2]) __attribute__((always_inline)) -> float {
    constexpr bool COPY = decltype(copy_tag)::value;
    const bool first = c_t == 0;
    wait_prev();
    __syncthreads();
    const int kb_next = kb_cur == 0 ? kKNB - 1 : kb_cur - 1;  // u % 3
    const int key0 = c_t * kBN;
    const bool slow = key0 + kBN > c_kv;
    if (COPY) {
      // the next item's q (items of two or more tiles) first: the waits
      // count the tile copies after it
      if (first && c_n > 1 && u + c_n < U) stage_q(c_e + 1);
      stage_clamped(vc.addr, a.vs[1], vc.rows, kVBuf + (vb_prev ^ 1) * kTileBytes);
      advance_copy(vc, v_addr, a.vs, v_tile_bytes);
      stage_clamped(kc.addr, a.ks[1], kc.rows, kKBuf + kb_next * kTileBytes);
      advance_copy(kc, k_addr, a.ks, k_tile_bytes);
    }
    float cc_ = c;
    if (slow) {  // the item's tail tile: keys from kv_end on -> -inf
      cc_ = 1.0f;
      const int hf4 = hf * 4;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int kbase = key0 + kb * 32 + g * 8 + hf4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float sv = S[kb][g * 4 + e] * c;
            S[kb][g * 4 + e] = kbase + e < c_kv ? sv : -__builtin_inff();
          }
        }
    }

    float l_tile = 0.f, alpha = 1.f;
    bool rare = false;
    {
      const lds_u8* kb0 = lds + kKBuf + kb_cur * kTileBytes;
      const lds_u8* vb0 = lds + kVBuf + vb_prev * kTileBytes;
      auto frag = [&](int s) __attribute__((always_inline)) -> bf16x8 {
        if (s < kPV) {
          const int db = s % kDB, j = (s / kDB) & 1, kb = s / (2 * kDB);
          const lds_u8* p = vb0 + (kb * 32 + 16 * j) * 128 + (db >> 1) * C::kHalfBytes;
          const int vo = voff[db & 1];
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + vo));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + 8 * 128 + (vo ^ 16)));
          return concat(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi));
        }
        const int ds = (s - kPV) >> 1, kb = (s - kPV) & 1;
        return *(const VX_LDS bf16x8*)(kb0 + kofs(ds & 3) + kb * 32 * 128 + (ds >> 2) * C::kHalfBytes);
      };
      const bf16x2 one2 = {(bf16)1.0f, (bf16)1.0f};
      if (!COPY) __builtin_amdgcn_s_setprio(1);
      bf16x8 fr[kSlots];
      float pf[32];
      bf16x2 pk[16];
      fr[0] = frag(0);
      fr[1] = frag(1);
      fr[2] = frag(2);
      auto softmax_block = [&]() __attribute__((always_inline)) {
        const float mneg = -m_run;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
          for (int i = 0; i < 8; ++i) pf[8 * g + i] = __builtin_fmaf(S[g >> 1][8 * (g & 1) + i], cc_, mneg);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < 8; ++i) pf[8 * g + i] = fast_exp2(pf[8 * g + i]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < 4; ++i) pk[4 * g + i] = bf16x2{(bf16)pf[8 * g + 2 * i], (bf16)pf[8 * g + 2 * i + 1]};
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) l_tile = __builtin_amdgcn_fdot2_f32_bf16(pk[i], one2, l_tile, false);
        __builtin_amdgcn_sched_barrier(0);
      };
      auto pack_p = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int q = kb * 8 + j * 4;
            P[kb][j] = __builtin_shufflevector(__builtin_shufflevector(pk[q], pk[q + 1], 0, 1, 2, 3),
                                               __builtin_shufflevector(pk[q + 2], pk[q + 3], 0, 1, 2, 3),
                                               0, 1, 2, 3, 4, 5, 6, 7);
          }
      };
      // rare path (not an item's first tile): the tile's probabilities
      // against its max, O and l_run rescaled to it. The copying waves take
      // it before their slots (the scores are then dead during the slots,
      // which keeps the kernel within its registers) and rescale O after
      // them; the results are the same.
      auto rare_path = [&]() __attribute__((always_inline)) {
        if (__builtin_amdgcn_ballot_w64(l_tile > kSumLimit || is_nan_bits(l_tile)) != 0) {
          rare = true;
          float mxc = -__builtin_inff();
#pragma unroll
          for (int e = 0; e < 16; ++e) mxc = __builtin_fmaxf(__builtin_fmaxf(mxc, S[0][e]), S[1][e]);
          const float mn = fmaxf(m_run, halves_max(mxc) * cc_);
          alpha = fast_exp2(m_run - mn);
          m_run = mn;
          l_run *= alpha;
          if (!COPY) {
#pragma unroll
            for (int db = 0; db < kDB; ++db) O[db] *= alpha;
          }
          l_tile = probs(S, cc_, m_run, P);
        }
      };
      // an item's first tile takes its max first (m_run = the rare path's
      // reference point for it), so that the speculative pass stands
      auto tile_probs = [&]() __attribute__((always_inline)) {
        if (first) {
          float mxc = -__builtin_inff();
#pragma unroll
          for (int e = 0; e < 16; ++e) mxc = __builtin_fmaxf(__builtin_fmaxf(mxc, S[0][e]), S[1][e]);
          m_run = fmaxf(kNegBig, halves_max(mxc) * cc_);
        }
        softmax_block();
        pack_p();
        rare_path();
      };
      if (COPY) tile_probs();
      Sn[0] = f32x16{};
      Sn[1] = f32x16{};
#pragma unroll
      for (int s = 0; s < kSlots; ++s) {
        if (s + 3 < kSlots) fr[s + 3] = frag(s + 3);
        if (s < kPV) {
          const int db = s % kDB, j = (s / kDB) & 1, kb = s / (2 * kDB);
          O[db] = mfma32x32x16(fr[s], Pp[kb][j], O[db]);
        } else {
          const int ds = (s - kPV) >> 1, kb = (s - kPV) & 1;
          Sn[kb] = mfma32x32x16(fr[s], qr[ds], Sn[kb]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (!COPY) __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      if (!COPY) tile_probs();
    }
    if (COPY && rare) {
#pragma unroll
      for (int db = 0; db < kDB; ++db) O[db] *= alpha;
    }
    kb_cur = kb_cur == kKNB - 1 ? 0 : kb_cur + 1;
    vb_prev ^= 1;
    return l_tile;
  };
  // Step u with the item changes around it: an item's first step resets the
  // reference point (and a one-tile item copies and loads the next item's q
  // first: its own QK^T slots score that item); after it, the previous
  // item's rows are stored and O restarts; after the step that scored the
  // item's last tile, the next item's q is loaded for the next step's slots.
  auto stream_step = [&](auto copy_tag, const int u, f32x16 (&S)[2], f32x16 (&Sn)[2],
                         const bf16x8 (&Pp)[2][2], bf16x8 (&P)[2][2]) __attribute__((always_inline)) {
    constexpr bool COPY = decltype(copy_tag)::value;
    const bool first = c_t == 0, last = c_t + 1 == c_n;
    if (first) {
      if (c_n == 1 && u + 1 < U) {
        if (COPY) {
          stage_q(c_e + 1);
          wait_vmem<0>();
        }
        __syncthreads();
        load_q(qr);
      }
    }
    const float l_tile = step(copy_tag, u, S, Sn, Pp, P);
    stored = first && has_prev;
    if (first) {
      if (has_prev) epilogue(c_e - 1, l_run);
#pragma unroll
      for (int db = 0; db < kDB; ++db) O[db] = f32x16{};
      l_run = l_tile;
    } else {
      l_run += l_tile;
    }
    if (c_t + 2 == c_n && u + 2 < U) {
      // (a two-tile item copied the next item's q in this step)
      if (first) {
        if (COPY) wait_vmem<0>();
        __syncthreads();
      }
      load_q(qr);
    }
    if (!last) {
      ++c_t;
    } else if (u + 1 < U) {
      has_prev = true;
      ++c_e;
      c_kv = entry(c_e).kv;
      c_n = tiles_of(c_kv);
      c_t = 0;
    }
  };

  f32x16 S2[2];
  bf16x8 P2[2][2];
  auto stream_loop = [&](auto copy_tag) __attribute__((always_inline)) {
    first_scores();
    int u = 0;
    for (; u + 1 < U; u += 2) {
      stream_step(copy_tag, u, S, S2, Pp, P2);
      stream_step(copy_tag, u + 1, S2, S, P2, Pp);
    }
    if (u < U) {
      stream_step(copy_tag, u, S, S2, Pp, P2);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) Pp[kb][j] = P2[kb][j];
    }
  };
  if (wave < kCopyWaves)
    stream_loop(std::integral_constant<bool, true>{});
  else
    stream_loop(std::integral_constant<bool, false>{});
  // ---- PV of the last tile (V buffer vb_prev) and the last item's rows
  wait_vmem<0>();
  __syncthreads();
  {
    const lds_u8* vb = lds + kVBuf + vb_prev * kTileBytes;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int db = 0; db < kDB; ++db) {
          const lds_u8* p = vb + (kb * 32 + 16 * j) * 128 + (db >> 1) * C::kHalfBytes;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + voff[db & 1]));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS s16x4*)(p + 8 * 128 + (voff[db & 1] ^ 16)));
          O[db] = mfma32x32x16(concat(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi)), Pp[kb][j],
                               O[db]);
        }
  }
  epilogue(c_e, l_run);
}

// Name of a flash_fwd_kernel instantiation, as the profiler prints it.
template <int MASK, int D, int WAVES>
const char* flash_kernel_name() {
  static const std::string name = "flash_fwd_kernel<" + std::to_string(MASK) + ", " + std::to_string(D) + ", " +
                                  std::to_string(WAVES) + ">";
  return name.c_str();
}

template <int MASK, int D, int WAVES>
const char* flash_split_kernel_name() {
  static const std::string name = "flash_fwd_split_kernel<" + std::to_string(MASK) + ", " + std::to_string(D) +
                                  ", " + std::to_string(WAVES) + ">";
  return name.c_str();
}

template <int MASK, int WAVES, int D>
int launch_one(const FlashArgs& a, hipStream_t stream, const char** launched) {
  const int n_qt = (a.Sq + WAVES * 32 - 1) / (WAVES * 32);
  if constexpr (!(MASK & (kMaskFull | kMaskBias))) {  // bias paths are not split
    if (a.split_items > 0) {
    const int n_items = n_qt * a.H * a.B;
    const int n_full = n_items - a.split_items;
    hipLaunchKernelGGL((flash_fwd_split_kernel<MASK, D, WAVES>), dim3(n_full + 2 * a.split_items),
                       dim3(WAVES * 64), 0, stream, a, n_full, n_qt);
    hipLaunchKernelGGL((flash_combine_kernel<D, WAVES>), dim3(a.split_items), dim3(WAVES * 64), 0, stream, a,
                       n_full, n_qt);
    *launched = flash_split_kernel_name<MASK, D, WAVES>();
    return (int)hipGetLastError();
    }
  }
  dim3 grid(n_qt, a.H, a.B);
  hipLaunchKernelGGL((flash_fwd_kernel<MASK, D, WAVES>), grid, dim3(WAVES * 64), 0, stream, a);
  *launched = flash_kernel_name<MASK, D, WAVES>();
  return (int)hipGetLastError();
}

template <int D>
const char* flash_stream_kernel_name() {
  static const std::string name = "flash_stream_kernel<" + std::to_string(D) + ">";
  return name.c_str();
}

// The persistent kernel: one workgroup per CU, a multiple of 8 (the XCDs).
// A workgroup's items start within 1/groups of the kernel's work (n + 3 per
// item of n <= T key tiles, T those of Sk: at most twice work = items *
// (T + 1)), and items with keys weigh at least 4, so it holds at most
// work / (2 * groups) + 1 of them;
// grids whose workgroups could exceed the LDS table run the 128-query
// kernel instead.
template <int D>
int launch_stream(const FlashArgs& a, hipStream_t stream, const char** launched) {
  const int groups = std::max(8, device_cu_count() / 8 * 8);
  const int64_t n_qt = (a.Sq + 255) / 256;
  const int64_t work = n_qt * a.H * a.B * ((a.Sk + kBN - 1) / kBN + 1);
  if (work / (2 * groups) + 2 > kStreamTabMax) return launch_one<kMaskNone, 4, D>(a, stream, launched);
  hipLaunchKernelGGL((flash_stream_kernel<D>), dim3(groups), dim3(512), 0, stream, a);
  *launched = flash_stream_kernel_name<D>();
  return (int)hipGetLastError();
}

// The workgroup size (4 or 8 waves) comes from the launch plan in a.waves,
// and a.stream picks the persistent kernel for short key sequences.
// (the per-(query, key) bias path, and key validity together with a key
// bias, always run 128-query workgroups)
template <int MASK>
int launch(const FlashArgs& a, hipStream_t stream, const char** launched) {
  if constexpr (MASK == kMaskNone) {
    if (a.stream)
      return a.D == 64 ? launch_stream<64>(a, stream, launched) : launch_stream<128>(a, stream, launched);
  }
  constexpr bool kOnly4 = (MASK & kMaskFull) || MASK == (kMaskValid | kMaskBias);
  if (a.waves == 4 || kOnly4)
    return a.D == 64 ? launch_one<MASK, 4, 64>(a, stream, launched) : launch_one<MASK, 4, 128>(a, stream, launched);
  if constexpr (!kOnly4)
    return a.D == 64 ? launch_one<MASK, 8, 64>(a, stream, launched) : launch_one<MASK, 8, 128>(a, stream, launched);
  return (int)hipErrorInvalidValue;
}

}  // namespace

// ---- scratch of the allocation-free entry point (vx_flash_attn_noalloc_fwd):
// the key-split partials live in this file-scope device array instead of a
// workspace. Each device that runs the library holds one copy until the
// process ends; calls on one device share it (their split launches must not
// overlap). kNoallocScratchBytes covers every split plan of a device with up
// to 262 compute units (the plan uses at most one partial slot per resident
// workgroup: 2 x 256 x 4 waves x 64 lanes x 66 floats = 33 MiB on MI355X).
constexpr int64_t kNoallocScratchBytes = 36ll << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

int noalloc_scratch(void** ptr, int64_t* bytes) {
  // device address of `scratch`, looked up once per device with that device
  // current (the host-side name is only a handle for the lookup)
  static std::mutex mu;
  static void* addr[64] = {nullptr};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    addr[dev] = p;
  }
  *ptr = addr[dev];
  *bytes = kNoallocScratchBytes;
  return 0;
}

int device_cu_count() {
  // per-device cache; host threads may race to fill an entry, each storing
  // the same value (relaxed atomics: no data race)
  static std::atomic<int> counts[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = counts[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    counts[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int launch_flash_fwd(const FlashArgs& a, void* stream, const char** launched) {
  if (a.D != 128 && a.D != 64) return (int)hipErrorNotSupported;
  if (a.waves != 4 && a.waves != 8) return (int)hipErrorInvalidValue;
  hipStream_t s = (hipStream_t)stream;
  const int mask = (a.key_valid != nullptr ? kMaskValid : 0) | (a.key_bias != nullptr ? kMaskBias : 0);
  if (a.full_bias != nullptr) {
    switch (mask) {
      case kMaskValid: return launch<kMaskFull | kMaskValid>(a, s, launched);
      case kMaskBias: return launch<kMaskFull | kMaskBias>(a, s, launched);
      case kMaskValid | kMaskBias: return launch<kMaskFull | kMaskValid | kMaskBias>(a, s, launched);
      default: return launch<kMaskFull>(a, s, launched);
    }
  }
  switch (mask) {
    case kMaskValid: return launch<kMaskValid>(a, s, launched);
    case kMaskBias: return launch<kMaskBias>(a, s, launched);
    case kMaskValid | kMaskBias: return launch<kMaskValid | kMaskBias>(a, s, launched);
    default: return launch<kMaskNone>(a, s, launched);
  }
}

}  // namespace vx
