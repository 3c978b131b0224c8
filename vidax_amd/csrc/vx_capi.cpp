// C ABI of the attention kernels (declared in include/vx_attn.h).
//
// Plain C++ with no HIP dependency: argument checks, error reporting and the
// failure-injection hook run on a host without a GPU. The kernels are reached
// through vx::launch_* (flash_fwd.hip, na3d_fwd.hip, qk_prologue.hip).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <cctype>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <string>

#include "../../include/vx_attn.h"
#include "vx_kernels.h"

namespace {

thread_local char g_error[512] = "";
thread_local const char* g_last_launch = "";
std::atomic<int32_t> g_inject{0};

int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int32_t ok() {
  g_error[0] = '\0';
  return VX_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Fills s[3] with the given strides or the contiguous (B, S, H, D) ones.
void strides_or_default(const int64_t* given, int32_t S, int32_t H, int32_t D, int64_t s[3]) {
  if (given != nullptr) {
    s[0] = given[0];
    s[1] = given[1];
    s[2] = given[2];
  } else {
    s[2] = D;
    s[1] = (int64_t)H * D;
    s[0] = (int64_t)S * H * D;
  }
}

int32_t check_strides(const char* name, const int64_t s[3], int32_t S) {
  for (int i = 0; i < 3; ++i) {
    if (s[i] < 0) return fail(VX_ERR_INVALID_ARGUMENT, "%s stride[%d] = %lld is negative", name, i, (long long)s[i]);
    if (s[i] % 8 != 0)
      return fail(VX_ERR_INVALID_ARGUMENT, "%s stride[%d] = %lld is not a multiple of 8 elements", name, i,
                  (long long)s[i]);
  }
  (void)S;  // row offsets are formed in 64-bit inside the kernels
  return VX_OK;
}

// ---- flash launch plan: the gfx950 tile table and its env override.
//
// Mirrors the reference's per-device tile table and VIDAX_FLASH_BLOCK_SIZES
// override (src/vidax/core/attention.py:10-35). Here a tile choice is the
// query tile of a workgroup: 128 queries (4 waves, two workgroups per CU)
// or 256 queries (8 waves, one per CU), with 64-key tiles either way. The
// library holds gfx950 code only, so the table has that one row.
struct FlashTileRule {
  const char* arch;
  int32_t max_seq_k_small;    // key sequences up to this run 128-query workgroups
  int64_t min_tiles_large;    // grids with fewer 256-query tiles run 128-query workgroups
  // ... except grids of at least this many 256-query tiles with no key
  // masks but kv_len, which run the persistent 256-query kernel
  int64_t min_tiles_stream;
};
constexpr FlashTileRule kFlashTileTable[] = {
    {"gfx950", 1024, 768, 4096},
};
constexpr int32_t kKeyTile = 64;

// VIDAX_FLASH_BLOCK_SIZES: "block_q,block_k_major,block_k" or "default"
// (the table's rule), read once per process.
struct FlashTileOverride {
  int32_t block_q = 0;  // 0: no override
  int32_t rc = VX_OK;   // non-zero: the variable is malformed or unsupported
  std::string error;
};

FlashTileOverride parse_tile_override(const char* env) {
  FlashTileOverride o;
  if (env == nullptr) return o;
  std::string v(env);
  while (!v.empty() && std::isspace((unsigned char)v.back())) v.pop_back();
  size_t b = 0;
  while (b < v.size() && std::isspace((unsigned char)v[b])) ++b;
  v = v.substr(b);
  if (v.empty()) return o;
  std::string lower = v;
  for (auto& ch : lower) ch = (char)std::tolower((unsigned char)ch);
  if (lower == "default") return o;
  long vals[3];
  const char* p = v.c_str();
  for (int i = 0; i < 3; ++i) {
    char* end = nullptr;
    vals[i] = std::strtol(p, &end, 10);
    while (*end == ' ') ++end;
    const char want = i < 2 ? ',' : '\0';
    if (end == p || *end != want) {
      o.rc = VX_ERR_INVALID_ARGUMENT;
      o.error = "VIDAX_FLASH_BLOCK_SIZES='" + v + "' must be 'block_q,block_k_major,block_k' or 'default'";
      return o;
    }
    p = end + (i < 2 ? 1 : 0);
  }
  if ((vals[0] != 128 && vals[0] != 256) || vals[1] != kKeyTile || vals[2] != kKeyTile) {
    o.rc = VX_ERR_UNSUPPORTED;
    o.error = "VIDAX_FLASH_BLOCK_SIZES='" + v +
              "': this build's flash kernel has query tiles of 128 or 256 and key tiles of 64 "
              "(e.g. '256,64,64')";
    return o;
  }
  o.block_q = (int32_t)vals[0];
  return o;
}

const FlashTileOverride& tile_override() {
  static std::once_flag once;
  static FlashTileOverride o;
  std::call_once(once, [] { o = parse_tile_override(std::getenv("VIDAX_FLASH_BLOCK_SIZES")); });
  return o;
}

// Workgroup size for a flash call: the override, else the table's rule. A
// per-(query, key) bias (the text encoders' short sequences) always runs
// 128-query workgroups.
// mask_kind bits: 1 key validity, 2 key bias, 4 per-(query, key) bias. The
// per-(query, key) bias (short text-encoder sequences) and key validity
// together with a key bias (a rare pair, which needs more registers than
// the 256-query kernel has without spilling) run 128-query workgroups.
//
// stream (optional): set to 1 when the plan picks the persistent 256-query
// kernel (key sequences up to max_seq_k_small, at least min_tiles_stream
// 256-query tiles, no key masks but kv_len, at most 64 batch items, few
// enough items per workgroup for its table). The override 128 turns it off;
// 256 keeps the rule.
int32_t flash_plan(int32_t B, int32_t Sq, int32_t Sk, int32_t H, int32_t mask_kind, int32_t* waves,
                   int32_t* stream = nullptr) {
  const FlashTileOverride& o = tile_override();
  if (o.rc != VX_OK) return fail(o.rc, "%s", o.error.c_str());
  if (stream != nullptr) *stream = 0;
  if ((mask_kind & 4) != 0 || (mask_kind & 3) == 3) {
    *waves = 4;
    return VX_OK;
  }
  const FlashTileRule& r = kFlashTileTable[0];
  const int64_t tiles256 = (int64_t)((Sq + 255) / 256) * H * B;
  const int64_t key_tiles = ((int64_t)Sk + kKeyTile - 1) / kKeyTile;
  const bool streamable = mask_kind == 0 && Sk <= r.max_seq_k_small && tiles256 >= r.min_tiles_stream && B <= 64 &&
                          tiles256 * (key_tiles + 1) / (2 * 256) + 2 <= vx::kStreamTabMax;
  if (o.block_q != 0) {
    *waves = o.block_q / 32;
    if (stream != nullptr) *stream = *waves == 8 && streamable ? 1 : 0;
    return VX_OK;
  }
  if (streamable) {
    *waves = 8;
    if (stream != nullptr) *stream = 1;
    return VX_OK;
  }
  *waves = (Sk <= r.max_seq_k_small || tiles256 < r.min_tiles_large) ? 4 : 8;
  return VX_OK;
}

void flash_kernel_label(int32_t mask_kind, int32_t D, int32_t waves, int32_t stream, char* out, int32_t len) {
  if (out == nullptr || len <= 0) return;
  if (stream)
    snprintf(out, (size_t)len, "flash_stream_kernel<%d>", D);
  else
    snprintf(out, (size_t)len, "flash_fwd_kernel<%d, %d, %d>", mask_kind, D, waves);
}

// ---- key split of the last round of a grid (vx_flash_attn_ws_fwd).
//
// A grid of n_items (query tile, head, batch) workgroups over `slots`
// resident workgroups (two 4-wave or one 8-wave workgroup per compute unit)
// runs ceil(n_items / slots) rounds; when the last round holds r <= slots/2
// items, running each of those as two workgroups over half the keys (and
// merging the halves) makes that round take half as long. Key sequences
// shorter than kMinSplitTiles key tiles are not split.
constexpr int32_t kMinSplitTiles = 16;

struct SplitPlan {
  int32_t items = 0;  // items split in two (0: none)
  int32_t k_mid = 0;  // first key of the second half (a multiple of the key tile)
  int64_t ws_bytes = 0;
};

SplitPlan flash_split_plan(int32_t B, int32_t Sq, int32_t Sk, int32_t H, int32_t D, int32_t waves,
                           int32_t num_cus) {
  SplitPlan p;
  const int64_t tiles = ((int64_t)Sk + kKeyTile - 1) / kKeyTile;
  if (num_cus <= 0 || tiles < kMinSplitTiles) return p;
  const int64_t n_qt = ((int64_t)Sq + waves * 32 - 1) / (waves * 32);
  const int64_t n_items = n_qt * H * B;
  const int64_t slots = (int64_t)num_cus * (waves == 4 ? 2 : 1);
  const int64_t rounds = (n_items + slots - 1) / slots;
  const int64_t r = n_items - (rounds - 1) * slots;
  if (r > slots / 2 || r > (1 << 20)) return p;
  p.items = (int32_t)r;
  p.k_mid = (int32_t)(tiles / 2 * kKeyTile);
  p.ws_bytes = 2 * r * vx::flash_part_floats(waves, D) * (int64_t)sizeof(float);
  return p;
}

// ---- neighbourhood-attention launch plan, by the clamped x window (and for
// head dim 64 with the tall bricks, the grid width: the 32-wide bricks when
// they leave no more ragged columns than the 16-wide ones).
//
// Head dim 64 with kw' <= 9 runs the tall 1 x 8 x 16 bricks (four waves per
// SIMD) unless they pad the y-x plane more than the 1 x 4 x 32 bricks do
// (same box, (3,7,7) and (3,5,5) windows: 5x22x40 NH=16 -10 %, 9x22x40 NH=8
// -6 %, 21x45x80 NH=24 -5 %, 17x44x80 NH=8 even; 5x11x20 NH=32, where the
// tall bricks cover 16 rows for 11, +37 %).
// Deep t windows (kt' >= kNaDeepMinKt) at head dim 64 with the 32-wide bricks
// take them two t planes deep: a wave's 2 x 4 x 4 queries need (kt' + 1) x
// (kh' + 3) key rows instead of the kt' x (kh' + 7) of 1 x 8 x 4.
int32_t na3d_variant(int32_t kt_clamped, int32_t kw_clamped, int32_t D, int32_t Hs, int32_t W) {
  if (kw_clamped <= 9) {
    const int64_t tall_area = (int64_t)((Hs + 7) / 8 * 8) * ((W + 15) / 16 * 16);
    const int64_t pipe_area = (int64_t)((Hs + 3) / 4 * 4) * ((W + 31) / 32 * 32);
    if (D == 64) return tall_area <= pipe_area ? vx::kNaTall : vx::kNaPipe16;
    return kt_clamped >= vx::kNaTStackMinKt ? vx::kNaTStack : vx::kNaPipe16;
  }
  if (kw_clamped <= 13) {
    if (D != 64 || (W + 31) / 32 * 32 != (W + 15) / 16 * 16) return vx::kNaTall;
    return kt_clamped >= vx::kNaDeepMinKt ? vx::kNaDeep : vx::kNaTallWide;
  }
  if (kw_clamped <= 25) return vx::kNaPipe32;
  return vx::kNaWave;
}

const char* na3d_kernel_label(int32_t variant, int32_t D) {
  switch (variant) {
    case vx::kNaPipe16: return D == 64 ? "na3d_pipe_kernel<16, 64>" : "na3d_pipe_kernel<16, 128>";
    case vx::kNaTall: return D == 64 ? "na3d_tall_kernel<64>" : "na3d_tall_kernel<128>";
    case vx::kNaTallWide: return "na3d_tall_wide_kernel<64>";
    case vx::kNaDeep: return "na3d_deep_kernel<64>";
    case vx::kNaTStack: return "na3d_tstack_kernel<128>";
    case vx::kNaPipe32: return D == 64 ? "na3d_pipe_kernel<32, 64>" : "na3d_pipe_kernel<32, 128>";
    default: return D == 64 ? "na3d_wave_kernel<64>" : "na3d_wave_kernel<128>";
  }
}

int32_t flash_check(const void* q, const void* k, const void* v, const void* out, const int32_t* kv_len,
                    const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride, int32_t B,
                    int32_t Sq, int32_t Sk,
                    int32_t H, int32_t D, const int64_t* qs_in, const int64_t* ks_in, const int64_t* vs_in,
                    const int64_t* os_in, float scale, vx::FlashArgs* args,
                    const float* full_bias = nullptr, const int64_t* fb_strides = nullptr) {
  (void)kv_len;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
    return fail(VX_ERR_INVALID_ARGUMENT, "q, k, v and out must be non-NULL");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(VX_ERR_INVALID_ARGUMENT, "q, k, v and out must be 16-byte aligned");
  if (B < 1 || Sq < 1 || Sk < 1 || H < 1)
    return fail(VX_ERR_INVALID_ARGUMENT, "batch (%d), seq_q (%d), seq_k (%d) and num_heads (%d) must be >= 1", B, Sq,
                Sk, H);
  if (B > 65535 || H > 65535)
    return fail(VX_ERR_INVALID_ARGUMENT, "batch (%d) and num_heads (%d) must be <= 65535", B, H);
  if (D != 128 && D != 64)
    return fail(VX_ERR_UNSUPPORTED, "head_dim %d is not supported (this build handles 64 and 128)", D);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(VX_ERR_INVALID_ARGUMENT, "scale must be positive and finite (got %g)", (double)scale);
  // a key bias enters the kernel's accumulator as bias / scale
  if (key_bias != nullptr && !std::isfinite(1.0f / scale))
    return fail(VX_ERR_INVALID_ARGUMENT, "scale %g is too small for a key bias (1/scale is not finite)",
                (double)scale);
  if (key_valid != nullptr || key_bias != nullptr) {
    const int64_t need = ((int64_t)Sk + 63) / 64 * 64;
    if (key_mask_stride < need || key_mask_stride % 4 != 0)
      return fail(VX_ERR_INVALID_ARGUMENT,
                  "key_mask_stride (%lld) must be a multiple of 4 and >= round_up(seq_k, 64) = %lld",
                  (long long)key_mask_stride, (long long)need);
    if (key_valid != nullptr && (reinterpret_cast<uintptr_t>(key_valid) & 3u) != 0)
      return fail(VX_ERR_INVALID_ARGUMENT, "key_valid must be 4-byte aligned");
    if (key_bias != nullptr && !aligned16(key_bias))
      return fail(VX_ERR_INVALID_ARGUMENT, "key_bias must be 16-byte aligned");
  }
  if (full_bias != nullptr) {
    if (!aligned16(full_bias)) return fail(VX_ERR_INVALID_ARGUMENT, "bias must be 16-byte aligned");
    if (fb_strides == nullptr) return fail(VX_ERR_INVALID_ARGUMENT, "bias_strides must be given with bias");
    for (int i = 0; i < 3; ++i)
      if (fb_strides[i] < 0 || fb_strides[i] % 4 != 0)
        return fail(VX_ERR_INVALID_ARGUMENT, "bias_strides[%d] = %lld must be a non-negative multiple of 4", i,
                    (long long)fb_strides[i]);
  }
  int64_t qs[3], ks[3], vs[3], os[3];
  strides_or_default(qs_in, Sq, H, D, qs);
  strides_or_default(ks_in, Sk, H, D, ks);
  strides_or_default(vs_in, Sk, H, D, vs);
  strides_or_default(os_in, Sq, H, D, os);
  int32_t rc;
  if ((rc = check_strides("q", qs, Sq)) != VX_OK) return rc;
  if ((rc = check_strides("k", ks, Sk)) != VX_OK) return rc;
  if ((rc = check_strides("v", vs, Sk)) != VX_OK) return rc;
  if ((rc = check_strides("out", os, Sq)) != VX_OK) return rc;
  // the kernel forms key-row offsets within a 64-key tile in 32 bits
  if (ks[1] > (int64_t(1) << 24) || vs[1] > (int64_t(1) << 24))
    return fail(VX_ERR_UNSUPPORTED, "k/v sequence strides (%lld, %lld) above 2^24 elements are not supported",
                (long long)ks[1], (long long)vs[1]);
  int32_t waves = 0, stream = 0;
  const int32_t mask_kind =
      (key_valid != nullptr ? 1 : 0) | (key_bias != nullptr ? 2 : 0) | (full_bias != nullptr ? 4 : 0);
  if ((rc = flash_plan(B, Sq, Sk, H, mask_kind, &waves, &stream)) != VX_OK) return rc;
  // the persistent kernel copies q tiles with 32-bit row offsets too, and
  // stores each 256-row block of the output through a buffer resource
  if (qs[1] > (int64_t(1) << 24) || os[1] > (int64_t(1) << 22)) stream = 0;
  if (args != nullptr) {
    args->waves = waves;
    args->stream = stream;
    args->split_items = 0;
    args->k_mid = 0;
    args->ws = nullptr;
    args->q = q;
    args->k = k;
    args->v = v;
    args->o = const_cast<void*>(out);
    args->kv_len = kv_len;
    args->key_valid = key_valid;
    args->key_bias = key_bias;
    args->key_mask_stride = key_mask_stride;
    args->B = B;
    args->Sq = Sq;
    args->Sk = Sk;
    args->H = H;
    args->D = D;
    for (int i = 0; i < 3; ++i) {
      args->qs[i] = qs[i];
      args->ks[i] = ks[i];
      args->vs[i] = vs[i];
      args->os[i] = os[i];
    }
    args->scale = scale;
    args->full_bias = full_bias;
    for (int i = 0; i < 3; ++i) args->fbs[i] = full_bias != nullptr ? fb_strides[i] : 0;
  }
  return ok();
}

int32_t na3d_check(const void* q, const void* k, const void* v, const void* out, int32_t B, int32_t T, int32_t Hs,
                   int32_t W, int32_t NH, int32_t D, int32_t kt, int32_t kh, int32_t kw, float scale,
                   vx::Na3dArgs* args) {
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
    return fail(VX_ERR_INVALID_ARGUMENT, "q, k, v and out must be non-NULL");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(VX_ERR_INVALID_ARGUMENT, "q, k, v and out must be 16-byte aligned");
  if (B < 1 || T < 1 || Hs < 1 || W < 1 || NH < 1)
    return fail(VX_ERR_INVALID_ARGUMENT, "batch (%d), t (%d), h (%d), w (%d) and num_heads (%d) must be >= 1", B, T, Hs,
                W, NH);
  if (kt < 1 || kh < 1 || kw < 1)
    return fail(VX_ERR_INVALID_ARGUMENT, "kernel sizes must be >= 1 (got %d, %d, %d)", kt, kh, kw);
  if (D != 128 && D != 64)
    return fail(VX_ERR_UNSUPPORTED, "head_dim %d is not supported (this build handles 64 and 128)", D);
  if (B > 65535 || NH > 65535)
    return fail(VX_ERR_INVALID_ARGUMENT, "batch (%d) and num_heads (%d) must be <= 65535", B, NH);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(VX_ERR_INVALID_ARGUMENT, "scale must be positive and finite (got %g)", (double)scale);
  const int64_t tokens = (int64_t)T * Hs * W;
  if (tokens * NH * D > ((int64_t)1 << 40))
    return fail(VX_ERR_INVALID_ARGUMENT, "tensor of %lld elements per batch item is too large",
                (long long)(tokens * NH * D));
  if ((int64_t)T * Hs * W > 0x7fffffff) return fail(VX_ERR_INVALID_ARGUMENT, "grid too large");
  if ((int64_t)W * NH * D >= ((int64_t)1 << 30))
    return fail(VX_ERR_UNSUPPORTED, "w x num_heads x head_dim = %lld elements per token row (must be below 2^30)",
                (long long)((int64_t)W * NH * D));
  if (args != nullptr) {
    args->q = q;
    args->k = k;
    args->v = v;
    args->o = const_cast<void*>(out);
    args->B = B;
    args->T = T;
    args->Hs = Hs;
    args->W = W;
    args->NH = NH;
    args->D = D;
    args->kt = kt < T ? kt : T;
    args->kh = kh < Hs ? kh : Hs;
    args->kw = kw < W ? kw : W;
    args->scale = scale;
    args->variant = na3d_variant(args->kt, args->kw, D, Hs, W);
    args->order = args->kt >= vx::kNaTColumnsMinKt ? vx::kNaOrderTColumns : vx::kNaOrderLaunch;
    args->q_prep = 0;
    args->q_weight = nullptr;
    args->q_cos = args->q_sin = nullptr;
    args->q_eps = 0.f;
    args->q_post_scale = 1.f;
    args->q_tab_stride = 0;
    args->q_ax_pairs[0] = args->q_ax_pairs[1] = 0;
  }
  return ok();
}

// The q-preparation arguments of vx_na3d_qprep_fwd, checked into a.
int32_t na3d_qprep_check(const float* weight, float eps, float post_scale, const float* rope_cos,
                         const float* rope_sin, int64_t rope_stride, int32_t D, vx::Na3dArgs* args) {
  int32_t prep = 0;
  if (weight != nullptr) {
    if (!aligned16(weight)) return fail(VX_ERR_INVALID_ARGUMENT, "q_norm_weight must be 16-byte aligned");
    if (!(eps >= 0.f) || !std::isfinite(eps))
      return fail(VX_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0 (got %g)", (double)eps);
    prep |= vx::kQPrepNorm;
  }
  if (!std::isfinite(post_scale))
    return fail(VX_ERR_INVALID_ARGUMENT, "q_post_scale must be finite (got %g)", (double)post_scale);
  if (post_scale != 1.0f) prep |= vx::kQPrepScale;
  if ((rope_cos == nullptr) != (rope_sin == nullptr))
    return fail(VX_ERR_INVALID_ARGUMENT, "rope_cos and rope_sin must both be given or both be NULL");
  if (rope_cos != nullptr) {
    if (!aligned16(rope_cos) || !aligned16(rope_sin))
      return fail(VX_ERR_INVALID_ARGUMENT, "rope_cos and rope_sin must be 16-byte aligned");
    if (rope_stride < D / 2 || rope_stride % 4 != 0)
      return fail(VX_ERR_INVALID_ARGUMENT, "rope_stride (%lld) must be a multiple of 4 and >= head_dim / 2 = %d",
                  (long long)rope_stride, D / 2);
    prep |= vx::kQPrepRope;
  }
  if (args != nullptr) {
    args->q_prep = prep;
    args->q_weight = weight;
    args->q_eps = eps;
    args->q_post_scale = post_scale;
    args->q_cos = rope_cos;
    args->q_sin = rope_sin;
    args->q_tab_stride = rope_stride;
    args->q_ax_pairs[0] = args->q_ax_pairs[1] = 0;
  }
  return VX_OK;
}

// The per-axis rotation table of vx_na3d_qprep_axes_fwd, checked into a:
// split (d_t, d_h, d_w) even, summing to head_dim, with d_t and d_h multiples
// of 8 (the kernel takes a lane's 4 pairs from one axis); 16-byte aligned
// cos/sin tables of t + h + w rows of rope_stride >= head_dim/2 floats (a
// multiple of 4), fewer than 2^31 elements (the kernel's offsets are 32-bit).
int32_t na3d_rope_axes_check(const float* cos, const float* sin, int64_t stride, const int32_t* split, int32_t D,
                             int32_t t, int32_t h, int32_t w, vx::Na3dArgs* args) {
  if (split == nullptr) {
    if (cos != nullptr || sin != nullptr) return fail(VX_ERR_INVALID_ARGUMENT, "rope tables need rope_split");
    return VX_OK;
  }
  for (int i = 0; i < 3; ++i)
    if (split[i] < 0 || split[i] % 2 != 0)
      return fail(VX_ERR_INVALID_ARGUMENT, "rope_split[%d] = %d must be even and >= 0", i, split[i]);
  if ((int64_t)split[0] + split[1] + split[2] != D)
    return fail(VX_ERR_INVALID_ARGUMENT, "rope_split (%d, %d, %d) must sum to head_dim %d", split[0], split[1],
                split[2], D);
  if (split[0] % 8 != 0 || split[1] % 8 != 0)
    return fail(VX_ERR_UNSUPPORTED, "rope_split (%d, %d, %d): the t and h parts must be multiples of 8", split[0],
                split[1], split[2]);
  if (cos == nullptr || sin == nullptr)
    return fail(VX_ERR_INVALID_ARGUMENT, "rope_split given without both rope_cos and rope_sin");
  if (!aligned16(cos) || !aligned16(sin))
    return fail(VX_ERR_INVALID_ARGUMENT, "rope_cos and rope_sin must be 16-byte aligned");
  if (stride < D / 2 || stride % 4 != 0)
    return fail(VX_ERR_INVALID_ARGUMENT, "rope_stride (%lld) must be a multiple of 4 and >= head_dim/2 = %d",
                (long long)stride, D / 2);
  if (((int64_t)t + h + w) * stride >= ((int64_t)1 << 31))
    return fail(VX_ERR_UNSUPPORTED, "rope tables of %lld rows x %lld floats exceed 2^31 elements",
                (long long)t + h + w, (long long)stride);
  if (args != nullptr) {
    args->q_prep |= vx::kQPrepRope | vx::kQPrepRopeAxes;
    args->q_cos = cos;
    args->q_sin = sin;
    args->q_tab_stride = stride;
    args->q_ax_pairs[0] = split[0] / 2;
    args->q_ax_pairs[1] = (split[0] + split[1]) / 2;
  }
  return VX_OK;
}

int32_t prologue_check(const void* x, const void* out, const float* weight, float eps, int32_t per_head,
                       float post_scale, const float* rope_cos, const float* rope_sin, int64_t rope_stride,
                       int32_t B, int32_t S, int32_t H, int32_t D, const int64_t* xs_in, const int64_t* os_in,
                       vx::PrologueArgs* args) {
  if (x == nullptr || out == nullptr) return fail(VX_ERR_INVALID_ARGUMENT, "x and out must be non-NULL");
  if (!std::isfinite(post_scale))
    return fail(VX_ERR_INVALID_ARGUMENT, "post_scale must be finite (got %g)", (double)post_scale);
  if (!aligned16(x) || !aligned16(out)) return fail(VX_ERR_INVALID_ARGUMENT, "x and out must be 16-byte aligned");
  if (B < 1 || S < 1 || H < 1)
    return fail(VX_ERR_INVALID_ARGUMENT, "batch (%d), seq (%d) and num_heads (%d) must be >= 1", B, S, H);
  if (D != 64 && D != 128)
    return fail(VX_ERR_UNSUPPORTED, "head_dim %d is not supported (this build handles 64 and 128)", D);
  if ((int64_t)H * D > 8192)
    return fail(VX_ERR_UNSUPPORTED, "rows of num_heads * head_dim = %lld exceed the supported 8192",
                (long long)H * D);
  if (per_head != 0 && per_head != 1) return fail(VX_ERR_INVALID_ARGUMENT, "per_head_norm must be 0 or 1");
  if (weight != nullptr) {
    if (!aligned16(weight)) return fail(VX_ERR_INVALID_ARGUMENT, "weight must be 16-byte aligned");
    if (!(eps >= 0.f) || !std::isfinite(eps))
      return fail(VX_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0 (got %g)", (double)eps);
  }
  if ((rope_cos == nullptr) != (rope_sin == nullptr))
    return fail(VX_ERR_INVALID_ARGUMENT, "rope_cos and rope_sin must both be given or both be NULL");
  if (rope_cos != nullptr) {
    if (!aligned16(rope_cos) || !aligned16(rope_sin))
      return fail(VX_ERR_INVALID_ARGUMENT, "rope_cos and rope_sin must be 16-byte aligned");
    if (rope_stride < D / 2 || rope_stride % 4 != 0)
      return fail(VX_ERR_INVALID_ARGUMENT, "rope_stride (%lld) must be a multiple of 4 and >= head_dim / 2 = %d",
                  (long long)rope_stride, D / 2);
  }
  const int64_t row = (int64_t)H * D;
  int64_t xs[2] = {S * row, row}, os[2] = {S * row, row};
  if (xs_in != nullptr) xs[0] = xs_in[0], xs[1] = xs_in[1];
  if (os_in != nullptr) os[0] = os_in[0], os[1] = os_in[1];
  for (int i = 0; i < 2; ++i) {
    if (xs[i] < 0 || xs[i] % 8 != 0 || os[i] < 0 || os[i] % 8 != 0)
      return fail(VX_ERR_INVALID_ARGUMENT, "strides must be non-negative multiples of 8 elements");
  }
  if (x == out && (xs[0] != os[0] || xs[1] != os[1]))
    return fail(VX_ERR_INVALID_ARGUMENT, "in-place use (out == x) needs identical strides");
  if (args != nullptr) {
    args->x = x;
    args->out = const_cast<void*>(out);
    args->weight = weight;
    args->cos = rope_cos;
    args->sin = rope_sin;
    args->eps = eps;
    args->post_scale = post_scale;
    args->per_head = per_head;
    args->B = B;
    args->S = S;
    args->H = H;
    args->D = D;
    args->x_bstride = xs[0];
    args->x_sstride = xs[1];
    args->o_bstride = os[0];
    args->o_sstride = os[1];
    args->tab_stride = rope_stride;
  }
  return ok();
}

int32_t injected() {
  const int32_t code = g_inject.load(std::memory_order_relaxed);
  if (code != 0) return fail(code, "error injected by vx_debug_inject_error(%d)", code);
  return VX_OK;
}

}  // namespace

extern "C" {

int32_t vx_abi_version(void) { return 10800; }

const char* vx_last_error(void) { return g_error; }

void vx_debug_inject_error(int32_t code) { g_inject.store(code, std::memory_order_relaxed); }

int32_t vx_debug_clock_stamp(uint64_t* out, int32_t n_groups, int32_t* wall_clock_khz, void* stream) {
  if (out == nullptr || wall_clock_khz == nullptr)
    return fail(VX_ERR_INVALID_ARGUMENT, "out and wall_clock_khz must be non-NULL");
  if ((reinterpret_cast<uintptr_t>(out) & 7u) != 0) return fail(VX_ERR_INVALID_ARGUMENT, "out must be 8-byte aligned");
  if (n_groups < 1 || n_groups > 4096) return fail(VX_ERR_INVALID_ARGUMENT, "n_groups must be in 1..4096");
  int khz = 0;
  const int err = vx::launch_clock_stamp(out, n_groups, stream, &khz);
  if (err != 0) return fail(VX_ERR_LAUNCH, "clock stamp launch failed (hipError_t %d)", err);
  *wall_clock_khz = khz;
  return ok();
}

const char* vx_last_launch(void) { return g_last_launch; }

int32_t vx_flash_attn_split_plan(int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                                 int32_t num_cus, int32_t* split_items, int32_t* split_key,
                                 int64_t* workspace_bytes) {
  if (batch < 1 || seq_q < 1 || seq_k < 1 || num_heads < 1)
    return fail(VX_ERR_INVALID_ARGUMENT, "batch, seq_q, seq_k and num_heads must be >= 1");
  if (head_dim != 128 && head_dim != 64)
    return fail(VX_ERR_UNSUPPORTED, "head_dim %d is not supported (this build handles 64 and 128)", head_dim);
  int32_t waves = 0, stream = 0;
  const int32_t rc = flash_plan(batch, seq_q, seq_k, num_heads, 0, &waves, &stream);
  if (rc != VX_OK) return rc;
  const SplitPlan p =
      stream ? SplitPlan{} : flash_split_plan(batch, seq_q, seq_k, num_heads, head_dim, waves, num_cus);
  if (split_items != nullptr) *split_items = p.items;
  if (split_key != nullptr) *split_key = p.k_mid;
  if (workspace_bytes != nullptr) *workspace_bytes = p.ws_bytes;
  return ok();
}

int64_t vx_flash_attn_workspace_size(int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads,
                                     int32_t head_dim) {
  int64_t bytes = 0;
  if (vx_flash_attn_split_plan(batch, seq_q, seq_k, num_heads, head_dim, vx::device_cu_count(), nullptr, nullptr,
                               &bytes) != VX_OK)
    return 0;
  return bytes;
}

int32_t vx_flash_attn_ws_fwd(const void* q, const void* k, const void* v, void* out, const int32_t* kv_len,
                             const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                             int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                             const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                             const int64_t* out_strides, float scale, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  vx::FlashArgs args;
  int32_t rc = flash_check(q, k, v, out, kv_len, key_valid, key_bias, key_mask_stride, batch, seq_q, seq_k,
                           num_heads, head_dim, q_strides, k_strides, v_strides, out_strides, scale, &args);
  if (rc != VX_OK) return rc;
  if (workspace_bytes < 0) return fail(VX_ERR_INVALID_ARGUMENT, "workspace_bytes must be >= 0");
  if (workspace != nullptr && !aligned16(workspace))
    return fail(VX_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  if ((rc = injected()) != VX_OK) return rc;
  // (calls with a key bias, and the persistent short-key kernel, are not split)
  const SplitPlan p = key_bias != nullptr || args.stream
                          ? SplitPlan{}
                          : flash_split_plan(batch, seq_q, seq_k, num_heads, head_dim, args.waves,
                                             vx::device_cu_count());
  if (p.items > 0 && workspace != nullptr && workspace_bytes >= p.ws_bytes) {
    args.split_items = p.items;
    args.k_mid = p.k_mid;
    args.ws = static_cast<float*>(workspace);
  }
  const char* launched = "";
  const int err = vx::launch_flash_fwd(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "flash attention launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

int32_t vx_flash_attn_plan(int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                           int32_t mask_kind, char* kernel_name, int32_t name_len) {
  if (batch < 1 || seq_q < 1 || seq_k < 1 || num_heads < 1)
    return fail(VX_ERR_INVALID_ARGUMENT, "batch, seq_q, seq_k and num_heads must be >= 1");
  if (head_dim != 128 && head_dim != 64)
    return fail(VX_ERR_UNSUPPORTED, "head_dim %d is not supported (this build handles 64 and 128)", head_dim);
  if (mask_kind < 0 || mask_kind > 7) return fail(VX_ERR_INVALID_ARGUMENT, "mask_kind must be in 0..7");
  int32_t waves = 0, stream = 0;
  const int32_t rc = flash_plan(batch, seq_q, seq_k, num_heads, mask_kind, &waves, &stream);
  if (rc != VX_OK) return rc;
  flash_kernel_label(mask_kind, head_dim, waves, stream, kernel_name, name_len);
  return ok();
}

int32_t vx_na3d_plan(int32_t t, int32_t h, int32_t w, int32_t head_dim, int32_t kernel_t, int32_t kernel_h,
                     int32_t kernel_w, char* kernel_name, int32_t name_len) {
  (void)kernel_h;
  const int32_t rc = na3d_check(reinterpret_cast<const void*>(16), reinterpret_cast<const void*>(16),
                                reinterpret_cast<const void*>(16), reinterpret_cast<const void*>(16), 1, t, h, w,
                                1, head_dim, kernel_t, kernel_h, kernel_w, 1.0f, nullptr);
  if (rc != VX_OK) return rc;
  const int32_t kw = kernel_w < w ? kernel_w : w;
  const int32_t kt = kernel_t < t ? kernel_t : t;
  if (kernel_name != nullptr && name_len > 0)
    snprintf(kernel_name, (size_t)name_len, "%s",
             na3d_kernel_label(na3d_variant(kt, kw, head_dim, h, w), head_dim));
  return ok();
}

int32_t vx_flash_attn_check(const void* q, const void* k, const void* v, const void* out, const int32_t* kv_len,
                            const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                            int32_t batch, int32_t seq_q,
                            int32_t seq_k, int32_t num_heads, int32_t head_dim, const int64_t* q_strides,
                            const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                            float scale) {
  return flash_check(q, k, v, out, kv_len, key_valid, key_bias, key_mask_stride, batch, seq_q, seq_k, num_heads,
                     head_dim,
                     q_strides, k_strides, v_strides, out_strides, scale, nullptr);
}

int32_t vx_flash_attn_fwd(const void* q, const void* k, const void* v, void* out, const int32_t* kv_len,
                          const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                          int32_t batch, int32_t seq_q,
                          int32_t seq_k, int32_t num_heads, int32_t head_dim, const int64_t* q_strides,
                          const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides, float scale,
                          void* stream) {
  vx::FlashArgs args;
  int32_t rc = flash_check(q, k, v, out, kv_len, key_valid, key_bias, key_mask_stride, batch, seq_q, seq_k,
                           num_heads, head_dim, q_strides, k_strides, v_strides, out_strides, scale, &args);
  if (rc != VX_OK) return rc;
  if ((rc = injected()) != VX_OK) return rc;
  const char* launched = "";
  const int err = vx::launch_flash_fwd(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "flash attention launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

int32_t vx_flash_attn_noalloc_fwd(const void* q, const void* k, const void* v, void* out, const int32_t* kv_len,
                                  const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                                  int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                                  const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* out_strides, float scale, void* stream) {
  vx::FlashArgs args;
  int32_t rc = flash_check(q, k, v, out, kv_len, key_valid, key_bias, key_mask_stride, batch, seq_q, seq_k,
                           num_heads, head_dim, q_strides, k_strides, v_strides, out_strides, scale, &args);
  if (rc != VX_OK) return rc;
  if ((rc = injected()) != VX_OK) return rc;
  const SplitPlan p = key_bias != nullptr || args.stream
                          ? SplitPlan{}
                          : flash_split_plan(batch, seq_q, seq_k, num_heads, head_dim, args.waves,
                                             vx::device_cu_count());
  if (p.items > 0) {
    void* ws = nullptr;
    int64_t cap = 0;
    const int err = vx::noalloc_scratch(&ws, &cap);
    if (err != 0) return fail(VX_ERR_LAUNCH, "looking up the static scratch failed (hipError_t %d)", err);
    if (p.ws_bytes > cap)
      return fail(VX_ERR_UNSUPPORTED,
                  "this shape splits its keys over %lld bytes of scratch; the static scratch holds %lld "
                  "(use vx_flash_attn_ws_fwd with a workspace)",
                  (long long)p.ws_bytes, (long long)cap);
    args.split_items = p.items;
    args.k_mid = p.k_mid;
    args.ws = static_cast<float*>(ws);
  }
  const char* launched = "";
  const int err = vx::launch_flash_fwd(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "flash attention launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

int32_t vx_flash_attn_bias_check(const void* q, const void* k, const void* v, const void* out, const int32_t* kv_len,
                                 const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                                 const float* bias, const int64_t* bias_strides, int32_t batch, int32_t seq_q,
                                 int32_t seq_k, int32_t num_heads, int32_t head_dim, const int64_t* q_strides,
                                 const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                                 float scale) {
  if (bias == nullptr) return fail(VX_ERR_INVALID_ARGUMENT, "bias must be non-NULL");
  return flash_check(q, k, v, out, kv_len, key_valid, key_bias, key_mask_stride, batch, seq_q, seq_k, num_heads,
                     head_dim, q_strides, k_strides, v_strides, out_strides, scale, nullptr, bias, bias_strides);
}

int32_t vx_flash_attn_bias_fwd(const void* q, const void* k, const void* v, void* out, const int32_t* kv_len,
                               const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                               const float* bias, const int64_t* bias_strides, int32_t batch, int32_t seq_q,
                               int32_t seq_k, int32_t num_heads, int32_t head_dim, const int64_t* q_strides,
                               const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                               float scale, void* stream) {
  if (bias == nullptr) return fail(VX_ERR_INVALID_ARGUMENT, "bias must be non-NULL");
  vx::FlashArgs args;
  int32_t rc = flash_check(q, k, v, out, kv_len, key_valid, key_bias, key_mask_stride, batch, seq_q, seq_k,
                           num_heads, head_dim, q_strides, k_strides, v_strides, out_strides, scale, &args, bias,
                           bias_strides);
  if (rc != VX_OK) return rc;
  if ((rc = injected()) != VX_OK) return rc;
  const char* launched = "";
  const int err = vx::launch_flash_fwd(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "flash attention launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

int32_t vx_na3d_check(const void* q, const void* k, const void* v, const void* out, int32_t batch, int32_t t,
                      int32_t h, int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t, int32_t kernel_h,
                      int32_t kernel_w, float scale) {
  return na3d_check(q, k, v, out, batch, t, h, w, num_heads, head_dim, kernel_t, kernel_h, kernel_w, scale, nullptr);
}

int32_t vx_na3d_fwd(const void* q, const void* k, const void* v, void* out, int32_t batch, int32_t t, int32_t h,
                    int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t, int32_t kernel_h,
                    int32_t kernel_w, float scale, void* stream) {
  vx::Na3dArgs args;
  int32_t rc = na3d_check(q, k, v, out, batch, t, h, w, num_heads, head_dim, kernel_t, kernel_h, kernel_w, scale,
                          &args);
  if (rc != VX_OK) return rc;
  if ((rc = injected()) != VX_OK) return rc;
  const char* launched = "";
  const int err = vx::launch_na3d_fwd(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "neighbourhood attention launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

int32_t vx_na3d_qprep_check(const void* q, const void* k, const void* v, const void* out, int32_t batch, int32_t t,
                            int32_t h, int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t,
                            int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight, float eps,
                            float q_post_scale, const float* rope_cos, const float* rope_sin, int64_t rope_stride) {
  int32_t rc = na3d_check(q, k, v, out, batch, t, h, w, num_heads, head_dim, kernel_t, kernel_h, kernel_w, 1.0f,
                          nullptr);
  if (rc != VX_OK) return rc;
  if ((rc = na3d_qprep_check(q_norm_weight, eps, q_post_scale, rope_cos, rope_sin, rope_stride, head_dim,
                             nullptr)) != VX_OK)
    return rc;
  return ok();
}

int32_t vx_na3d_qprep_fwd(const void* q, const void* k, const void* v, void* out, int32_t batch, int32_t t,
                          int32_t h, int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t,
                          int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight, float eps,
                          float q_post_scale, const float* rope_cos, const float* rope_sin, int64_t rope_stride,
                          void* stream) {
  vx::Na3dArgs args;
  int32_t rc = na3d_check(q, k, v, out, batch, t, h, w, num_heads, head_dim, kernel_t, kernel_h, kernel_w, 1.0f,
                          &args);
  if (rc != VX_OK) return rc;
  if ((rc = na3d_qprep_check(q_norm_weight, eps, q_post_scale, rope_cos, rope_sin, rope_stride, head_dim,
                             &args)) != VX_OK)
    return rc;
  if ((rc = injected()) != VX_OK) return rc;
  const char* launched = "";
  const int err = vx::launch_na3d_fwd(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "neighbourhood attention launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

int32_t vx_na3d_qprep_axes_check(const void* q, const void* k, const void* v, const void* out, int32_t batch,
                                 int32_t t, int32_t h, int32_t w, int32_t num_heads, int32_t head_dim,
                                 int32_t kernel_t, int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight,
                                 float eps, float q_post_scale, const float* rope_cos, const float* rope_sin,
                                 int64_t rope_stride, const int32_t* rope_split) {
  int32_t rc = na3d_check(q, k, v, out, batch, t, h, w, num_heads, head_dim, kernel_t, kernel_h, kernel_w, 1.0f,
                          nullptr);
  if (rc != VX_OK) return rc;
  if ((rc = na3d_qprep_check(q_norm_weight, eps, q_post_scale, nullptr, nullptr, 0, head_dim, nullptr)) != VX_OK)
    return rc;
  if ((rc = na3d_rope_axes_check(rope_cos, rope_sin, rope_stride, rope_split, head_dim, t, h, w, nullptr)) != VX_OK)
    return rc;
  return ok();
}

int32_t vx_na3d_qprep_axes_fwd(const void* q, const void* k, const void* v, void* out, int32_t batch, int32_t t,
                               int32_t h, int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t,
                               int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight, float eps,
                               float q_post_scale, const float* rope_cos, const float* rope_sin, int64_t rope_stride,
                               const int32_t* rope_split, void* stream) {
  vx::Na3dArgs args;
  int32_t rc = na3d_check(q, k, v, out, batch, t, h, w, num_heads, head_dim, kernel_t, kernel_h, kernel_w, 1.0f,
                          &args);
  if (rc != VX_OK) return rc;
  if ((rc = na3d_qprep_check(q_norm_weight, eps, q_post_scale, nullptr, nullptr, 0, head_dim, &args)) != VX_OK)
    return rc;
  if ((rc = na3d_rope_axes_check(rope_cos, rope_sin, rope_stride, rope_split, head_dim, t, h, w, &args)) != VX_OK)
    return rc;
  if ((rc = injected()) != VX_OK) return rc;
  const char* launched = "";
  const int err = vx::launch_na3d_fwd(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "neighbourhood attention launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

int32_t vx_rmsnorm_rope_check(const void* x, const void* out, const float* weight, float eps, int32_t per_head_norm,
                              const float* rope_cos, const float* rope_sin, int64_t rope_stride, int32_t batch,
                              int32_t seq, int32_t num_heads, int32_t head_dim, const int64_t* x_strides,
                              const int64_t* out_strides) {
  return prologue_check(x, out, weight, eps, per_head_norm, 1.0f, rope_cos, rope_sin, rope_stride, batch, seq,
                        num_heads, head_dim, x_strides, out_strides, nullptr);
}

int32_t vx_rmsnorm_rope_fwd(const void* x, void* out, const float* weight, float eps, int32_t per_head_norm,
                            const float* rope_cos, const float* rope_sin, int64_t rope_stride, int32_t batch,
                            int32_t seq, int32_t num_heads, int32_t head_dim, const int64_t* x_strides,
                            const int64_t* out_strides, void* stream) {
  return vx_rmsnorm_scale_rope_fwd(x, out, weight, eps, per_head_norm, 1.0f, rope_cos, rope_sin, rope_stride, batch,
                                   seq, num_heads, head_dim, x_strides, out_strides, stream);
}

int32_t vx_rmsnorm_scale_rope_check(const void* x, const void* out, const float* weight, float eps,
                                    int32_t per_head_norm, float post_scale, const float* rope_cos,
                                    const float* rope_sin, int64_t rope_stride, int32_t batch, int32_t seq,
                                    int32_t num_heads, int32_t head_dim, const int64_t* x_strides,
                                    const int64_t* out_strides) {
  return prologue_check(x, out, weight, eps, per_head_norm, post_scale, rope_cos, rope_sin, rope_stride, batch, seq,
                        num_heads, head_dim, x_strides, out_strides, nullptr);
}

int32_t vx_rmsnorm_scale_rope_fwd(const void* x, void* out, const float* weight, float eps, int32_t per_head_norm,
                                  float post_scale, const float* rope_cos, const float* rope_sin,
                                  int64_t rope_stride, int32_t batch, int32_t seq, int32_t num_heads,
                                  int32_t head_dim, const int64_t* x_strides, const int64_t* out_strides,
                                  void* stream) {
  vx::PrologueArgs args;
  int32_t rc = prologue_check(x, out, weight, eps, per_head_norm, post_scale, rope_cos, rope_sin, rope_stride, batch,
                              seq, num_heads, head_dim, x_strides, out_strides, &args);
  if (rc != VX_OK) return rc;
  if ((rc = injected()) != VX_OK) return rc;
  const char* launched = "";
  const int err = vx::launch_qk_prologue(args, stream, &launched);
  if (err != 0) return fail(VX_ERR_LAUNCH, "rmsnorm/rope launch failed (hipError_t %d)", err);
  g_last_launch = launched;
  return ok();
}

}  // extern "C"
