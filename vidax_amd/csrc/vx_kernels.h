// Internal interface between the C ABI (vx_capi.cpp, plain C++) and the HIP
// launchers (*.hip). No HIP headers here so the argument checker builds and
// runs on a host without a GPU.
#pragma once

#include <stdint.h>

namespace vx {

// Flash attention launch arguments, validated by the C ABI before use.
// Strides are in elements: {batch, seq, head}; the head dim is contiguous.
struct FlashArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* kv_len;     // [B] or nullptr
  const uint8_t* key_valid;  // [B, key_mask_stride] or nullptr
  const float* key_bias;     // [B, key_mask_stride] or nullptr
  int64_t key_mask_stride;   // elements between batch rows of the key masks
  const float* full_bias;    // [b*fbs[0] + h*fbs[1] + q*fbs[2] + key] or nullptr
  int64_t fbs[3];            // full-bias strides (elements) for batch, head, query
  int32_t B, Sq, Sk, H, D;
  int64_t qs[3], ks[3], vs[3], os[3];
  float scale;  // softmax scale (> 0)
  int32_t waves;  // workgroup size chosen by the launch plan: 4 (128 queries) or 8 (256)
  // 1: the persistent 256-query kernel for short key sequences (waves 8, no
  // key masks but kv_len, no key split), chosen by the launch plan
  int32_t stream;
  // Key split chosen by the launch plan (split_items = 0: none): each of the
  // last split_items (query tile, head, batch) items runs as two workgroups
  // over keys [0, k_mid) and [k_mid, Sk), writing fp32 partials to ws
  // (flash_part_floats floats per workgroup), merged by a second kernel.
  int32_t split_items;
  int32_t k_mid;
  float* ws;
};

// Items (with keys) one workgroup of the persistent short-key kernel holds
// in its LDS table. A workgroup's items start within 1/groups of the
// kernel's work (key tiles + 3 per item, at most twice work = items * (T +
// 1) with T the key tiles of Sk), and items with keys weigh at least 4, so
// it holds at most work / (2 * groups) + 1 of them: the plan picks the kernel only for
// grids with work / (2 * 256) + 2 <= kStreamTabMax, and the launcher checks
// the same with the device's workgroup count.
constexpr int kStreamTabMax = 1024;

// fp32 values of one key-split partial: the lanes' O accumulators, then
// (reference point, row sum) per lane.
constexpr int64_t flash_part_floats(int waves, int head_dim) {
  return (int64_t)waves * 64 * ((head_dim / 32) * 16 + 2);
}

// Neighbourhood attention launch arguments; tensors are contiguous
// (B, T, Hs, W, NH, D).
struct Na3dArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int32_t B, T, Hs, W, NH, D;
  int32_t kt, kh, kw;  // window sizes already clamped to the grid extents
  float scale;
  int32_t variant;     // kernel chosen by the launch plan (Na3dVariant)
  int32_t order;       // brick order of the pipelined kernels (Na3dOrder), chosen by the launch plan
  // q preparation applied by the kernel as it loads q (0 = q is used as
  // given): bit 1 per-head RMSNorm with q_weight[D] and q_eps, bit 2 times
  // bf16(q_post_scale), bit 4 rotation of adjacent pairs by the token's
  // (q_cos, q_sin) row (token t*Hs*W + y*W + x, D/2 fp32 values at
  // q_tab_stride)
  int32_t q_prep;
  const float* q_weight;
  float q_eps;
  float q_post_scale;
  const float* q_cos;
  const float* q_sin;
  int64_t q_tab_stride;
  // bit 8 (with 4): q_cos / q_sin hold per-axis rows instead, T rows of the
  // t axis, then Hs of the h axis, then W of the w axis (q_tab_stride
  // apart, fewer than 2^31 elements): pair j < q_ax_pairs[0] of token
  // (t, y, x) is read at column j of row t, j < q_ax_pairs[1] of row T + y,
  // the rest of row T + Hs + x; the boundaries are multiples of 4
  int32_t q_ax_pairs[2];
};
constexpr int32_t kQPrepNorm = 1, kQPrepScale = 2, kQPrepRope = 4, kQPrepRopeAxes = 8;

// Neighbourhood-attention kernels, by the clamped x window kw' and head dim.
enum Na3dVariant : int32_t {
  kNaPipe16 = 0,  // kw' <= 9: row streaming, 16-key x segments, 1 x 4 x 32 bricks
  kNaTall = 1,    // 9 < kw' <= 13: the same body on 1 x 8 x 16 bricks
  kNaPipe32 = 2,  // 13 < kw' <= 25: 32-key x segments
  kNaWave = 3,    // 25 < kw' <= 57, head dim 128: per-wave bricks
  kNaTallWide = 4,  // head dim 64, 9 < kw' <= 13, round_up(W, 32) == round_up(W, 16): 1 x 8 x 32 bricks
  kNaDeep = 5,      // as kNaTallWide with kt' >= kNaDeepMinKt: 2 x 4 x 32 bricks
  kNaTStack = 6,    // as kNaPipe16 at head dim 128 with kt' >= kNaTStackMinKt: 2 x 4 x 16 bricks
};
// t windows (clamped) from which the plan takes the t-stacked bricks
constexpr int32_t kNaTStackMinKt = 2;
// t windows (clamped) from which the plan takes the deep bricks
constexpr int32_t kNaDeepMinKt = 5;

// Order in which the pipelined NA kernels' workgroups take their bricks.
enum Na3dOrder : int32_t {
  kNaOrderLaunch = 0,    // launch order (heads spread over the XCDs when NH % 8 == 0)
  kNaOrderTColumns = 1,  // each XCD walks consecutive t planes of brick columns (deep t windows)
};
// t windows (clamped) from which the plan picks kNaOrderTColumns: bricks of
// consecutive t planes then share kt' - 1 of their kt' key planes in an L2
constexpr int32_t kNaTColumnsMinKt = 5;

struct PrologueArgs {
  const void* x;        // bf16 rows of H * D
  void* out;            // bf16, same row layout
  const float* weight;  // H * D (whole-row norm) or H * D (per-head norm, per channel); NULL = no norm
  const float* cos;     // (S, >= D/2) rows at tab_stride; NULL = no rotation
  const float* sin;
  float eps;
  float post_scale;     // 1: none; else y = bf16(y * bf16(post_scale)) after the norm
  int32_t per_head;     // 0: mean over the whole row, 1: over each head
  int32_t B, S, H, D;
  int64_t x_bstride, x_sstride, o_bstride, o_sstride, tab_stride;  // elements
};

// Compute units of the current device (0 if unknown), cached per device.
int device_cu_count();

// Device address and size of the current device's static scratch array
// (used by vx_flash_attn_noalloc_fwd); returns a hipError_t value.
int noalloc_scratch(void** ptr, int64_t* bytes);

// All return a hipError_t value (0 on success) and store the name of the kernel they launched in *launched (a string with
// static storage, built from the launched instantiation's template
// arguments).
int launch_flash_fwd(const FlashArgs& a, void* stream, const char** launched);
int launch_na3d_fwd(const Na3dArgs& a, void* stream, const char** launched);
int launch_qk_prologue(const PrologueArgs& a, void* stream, const char** launched);

// Measurement only: n_groups one-wave workgroups each store (XCD id, HW_ID,
// shader clock counter, real-time counter) as four uint64 at out + 4 * group;
// *wall_clock_khz receives the real-time counter's rate.
int launch_clock_stamp(uint64_t* out, int n_groups, void* stream, int* wall_clock_khz);

}  // namespace vx
