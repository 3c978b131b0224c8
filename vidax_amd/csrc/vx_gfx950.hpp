// gfx950 (CDNA4) building blocks shared by the attention kernels: vector
// types, the bf16 MFMA, the LDS transpose read, cross-half lane exchange, the
// exp2 used by the softmax, the LDS bank swizzle and the HBM -> LDS DMA copies.
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

#include <type_traits>

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

// Output rows of a wave's O^T accumulators (C layout above: lane l holds
// column l%32 = one query, element 4g+e of block db = d db*32 + 8g +
// (l/32)*4 + e), normalised by inv and packed to bf16 as 16-byte chunks:
// one v_permlane32_swap per dword trades 4-d chunks between the half waves,
// so that chunk (db, pr) of lane l holds d db*32 + 8*(2pr + l/32) + 0..7 of
// its query. All 64 lanes must be active.
template <int kDB>
__device__ __forceinline__ void pack_out_rows(const f32x16 (&O)[kDB], float inv, u32x4 (&chunk)[kDB][2]) {
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      bf16x4 lo, hi;  // d groups g = 2pr (lo) and 2pr + 1 (hi), 4 d each
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = (bf16)(O[db][8 * pr + e] * inv);
        hi[e] = (bf16)(O[db][8 * pr + 4 + e] * inv);
      }
      u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const auto r = __builtin_amdgcn_permlane32_swap(a[w], b[w], false, false);
        a[w] = r[0];
        b[w] = r[1];
      }
      chunk[db][pr] = u32x4{a[0], a[1], b[0], b[1]};
    }
}

// Regroups the packed output chunks of two 32-wide d blocks (c[b][pr] as
// pack_out_rows leaves them for blocks 2p + b) into whole 128-byte lines:
// out[i] of lane l holds 8-d chunk ((l >> 4) & 1) * 2 + (l >> 5) of block
// 2p + ((l >> 3) & 1) of the wave's query row (l & 7) + 8 i, so that a
// 16-byte store of out[i] per lane writes 8 rows x 128 contiguous bytes
// (instead of 32 rows x 32 bytes). Per dword one v_permlane16_swap trades
// chunks between 16-lane rows (pr 0 of rows 1 and 3 with pr 1 of rows 0 and
// 2: lane l then holds row l & 15, then l & 15 + 16) and two DPP moves
// rotate the 16-lane rows by 8 under a bank mask (rows 0-7 of both blocks,
// then rows 8-15). All 64 lanes must be active.
__device__ __forceinline__ void line_chunks(u32x4 (&c)[2][2], u32x4 (&out)[4]) {
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const auto r = __builtin_amdgcn_permlane16_swap(c[b][0][w], c[b][1][w], false, false);
      c[b][0][w] = r[0];
      c[b][1][w] = r[1];
    }
  constexpr int kRowRor8 = 0x128;  // DPP row_ror:8
#pragma unroll
  for (int xy = 0; xy < 2; ++xy)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      // lanes 8-15 of each row (banks 2, 3) take block 1 of the row 8 lanes down
      out[2 * xy][w] = __builtin_amdgcn_update_dpp(c[0][xy][w], c[1][xy][w], kRowRor8, 0xf, 0xc, false);
      // lanes 0-7 (banks 0, 1) take block 0 of the row 8 lanes up
      out[2 * xy + 1][w] = __builtin_amdgcn_update_dpp(c[1][xy][w], c[0][xy][w], kRowRor8, 0xf, 0x3, false);
    }
}

// Byte offset, within its row, of the chunk line_chunks leaves in lane l
// for the block pair p.
__device__ __forceinline__ uint32_t line_chunk_offset(int lane, int p) {
  return (uint32_t)((2 * p + ((lane >> 3) & 1)) * 64 + (((lane >> 4) & 1) * 2 + (lane >> 5)) * 16);
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

// XOR swizzle of the 16-byte chunk index (0-7) within the 128-byte half row
// of key (or key slot) r: the bit reversal of (r >> 1) & 7. The LDS has 64 four-byte banks
// (256 bytes per cycle) and two consecutive half rows cover them once, so
//  - the K reads (ds_read_b128, 16 lanes = keys 16i..16i+15 per cycle, one
//    chunk index) hit 16 distinct 16-byte bank groups: the 8 even and the 8
//    odd keys each see all 8 swizzles;
//  - the V transpose reads (ds_read_b64_tr_b16, 32 lanes = keys 4i..4i+3,
//    four chunks each, per cycle) hit 16 distinct groups: keys 4i, 4i+2 (and
//    4i+1, 4i+3) differ in bit 2 of the swizzle.
// Keys r and r + 8 differ only in bit 0 of the swizzle.
__device__ __forceinline__ int half_swizzle(int r) {
  return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
}

// One LDS DMA copy: 16 bytes per lane from `src` to LDS byte address
// lds_row + 16 * lane (LDS base in M0). Issued as inline assembly so the
// compiler does not treat every later LDS read as a possible reader of this
// write (it would wait for the copy to land before the first such read); the
// kernel orders each copy itself with wait_vmem + a barrier before any wave
// reads the destination buffer.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_row) {
  // M0 (the LDS destination) is set inside the statement and declared
  // clobbered; the compiler places no other M0 access in these kernels
  // (none appears in their assembly), so nothing of its own is lost. One
  // wait state separates the M0 write from the LDS DMA that reads it.
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_row))
               : "memory", "m0");
}

// Raw buffer resource over [base, base + 4 GiB): no stride, untyped 32-bit
// data, no range limit in practice (every offset used is below 2^31).
typedef int i32x4_rsrc __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4_rsrc raw_rsrc(const void* base) {
  const uint64_t addr = (uint64_t)(uintptr_t)base;
  // the base is uniform: keep the resource in scalar registers
  i32x4_rsrc r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32));  // 48-bit address; stride field 0
  r[2] = -1;                                                            // num_records
  r[3] = 0x00020000;                                                    // data format 32, raw access
  return r;
}

// A wave-uniform 64-bit value moved to scalar registers, so that address
// arithmetic on it stays on the scalar unit.
__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// raw_rsrc from a wave-uniform byte address (kept in scalar registers).
__device__ __forceinline__ i32x4_rsrc raw_rsrc_u64(uint64_t addr) {
  i32x4_rsrc r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32));
  r[2] = -1;
  r[3] = 0x00020000;
  return r;
}

// The same copy from a buffer resource: lane L fetches 16 bytes at byte
// offset voff. A 32-bit offset per lane (not a 64-bit address) makes the
// instruction cheaper to issue.
__device__ __forceinline__ void lds_dma16_buf(i32x4_rsrc rsrc, uint32_t voff, uint32_t lds_row) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(lds_row))
               : "memory", "m0");
}

// lds_dma16_buf with a scalar byte offset added to every lane's offset.
__device__ __forceinline__ void lds_dma16_buf_so(i32x4_rsrc rsrc, uint32_t voff, uint32_t soff, uint32_t lds_row) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "s"(__builtin_amdgcn_readfirstlane(lds_row))
               : "memory", "m0");
}

// s_waitcnt vmcnt(N), other counters untouched.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// NaN test on the bit pattern (stays exact when the compiler may assume no NaNs).
__device__ __forceinline__ bool is_nan_bits(float x) { return (__float_as_uint(x) & 0x7fffffffu) > 0x7f800000u; }

}  // namespace vx
