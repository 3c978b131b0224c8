/*
 * vx_attn.h -- C ABI of the MI355X (gfx950) attention kernels.
 *
 * Plain C: pointers, sizes and a HIP stream passed as an opaque pointer. No
 * framework types cross this boundary. Every entry point returns VX_OK (0) or
 * a non-zero VX_ERR_* code; the message for the last failure on the calling
 * thread is available from vx_last_error(). Nothing throws across the ABI.
 *
 * Layouts are the reference's: q/k/v/out are (B, S, H, D) bf16 for the flash
 * entry point and (B, T, Hs, W, NH, D) bf16 for the neighbourhood entry
 * point, with D (the head dim) contiguous. The library allocates nothing,
 * keeps no pointer after returning and never synchronises the stream. Every
 * entry point may be called concurrently from several host threads, except
 * vx_flash_attn_noalloc_fwd: its calls share one static scratch array per
 * device, so calls of it that overlap on one device race (see there).
 */
#ifndef VX_ATTN_H_
#define VX_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VX_OK 0
#define VX_ERR_INVALID_ARGUMENT 1 /* shape, stride, alignment, dtype or window error */
#define VX_ERR_UNSUPPORTED 2      /* a valid request this build has no kernel for   */
#define VX_ERR_LAUNCH 3           /* the HIP runtime refused the launch             */

/* Version of this ABI (major * 10000 + minor * 100 + patch): 1.8.0. */
int32_t vx_abi_version(void);

/* Message describing the most recent failure on the calling thread ("" if none). */
const char* vx_last_error(void);

/*
 * Non-causal flash attention forward:
 *   out[b, i, h, :] = sum_j softmax_j(scale * q[b,i,h,:] . k[b,j,h,:] + mask_bj) v[b, j, h, :]
 * with fp32 softmax statistics and fp32 accumulation, bf16 in and out.
 *
 * Replaces the reference's flash-attention call sites:
 *   - src/vidax/core/attention.py:212-288  (_flash_attention_tpu: q/k/v (B,S,H,D),
 *     sm_scale, zero-padded tails excluded through segment ids at :272-278)
 *   - src/vidax/core/attention.py:321-338  (local_attention)
 *   - src/vidax/core/attention.py:467-533  (dot_product_attention, flash branch)
 *   - src/vidax/models/hunyuan_video/common/dit_layers.py:150-190
 *     (_flash_attention_tpu_segment_masked: key-only validity mask)
 *
 * Key masking (all optional and combined; every one is key-only, i.e. the
 * same for every query row and every head of a batch item):
 *   kv_len     int32[B] or NULL: keys j >= kv_len[b] are masked (prefix form,
 *              the Hunyuan `key_valid` layout; values are clamped to [0, Sk]).
 *              It also bounds the key loop, so masked tails cost nothing.
 *   key_valid  uint8[B, key_mask_stride] or NULL: key j of batch b is valid
 *              iff key_valid[b*key_mask_stride + j] != 0 (general form).
 *   key_bias   float32[B, key_mask_stride] or NULL: added to the logits of
 *              key j after scaling; -inf masks the key (Cosmos3's
 *              (B,1,1,Sk) bias, src/vidax/models/cosmos3/dit_layers.py:124-135).
 * key_mask_stride is in elements, a multiple of 4 and >= round_up(Sk, 64) (the
 * kernel stages whole 64-key tiles of the mask; padding entries are not read
 * as keys);
 * key_valid must be 4-byte and key_bias 16-byte aligned.
 * A query row whose keys are all masked produces an all-zero output row.
 *
 * Strides (element units, {batch, seq, head}) may be NULL for a contiguous
 * (B, S, H, D) tensor; the head dim must be contiguous. q/k/v/out must be
 * 16-byte aligned and every stride a multiple of 8 elements.
 * Supported: head_dim 64 or 128, scale > 0 and finite, 1 <= B, H <= 65535,
 * 1 <= Sq, Sk < 2^31, k and v sequence strides <= 2^24 elements.
 * `stream` is a hipStream_t (NULL = the default stream).
 */
int32_t vx_flash_attn_fwd(const void* q, const void* k, const void* v, void* out,
                          const int32_t* kv_len, const uint8_t* key_valid,
                          const float* key_bias, int64_t key_mask_stride,
                          int32_t batch, int32_t seq_q,
                          int32_t seq_k, int32_t num_heads, int32_t head_dim,
                          const int64_t* q_strides, const int64_t* k_strides,
                          const int64_t* v_strides, const int64_t* out_strides, float scale,
                          void* stream);

/*
 * vx_flash_attn_fwd with a caller-provided device workspace (no other
 * argument differs). When a grid's last round of workgroups would leave
 * most of the device idle (e.g. 732 workgroups of 128 queries over 512
 * resident ones), the query tiles of that round are each computed as two
 * workgroups over the two halves of the keys, whose fp32 partial results go
 * to the workspace and are merged by a second kernel on the same stream.
 * That needs vx_flash_attn_workspace_size() bytes (0: no split for this
 * shape on this device); with a smaller workspace (or NULL), or with a
 * key_bias, the call runs without the split, as vx_flash_attn_fwd. The workspace must be 16-byte
 * aligned and stay untouched until the work on `stream` has finished; calls
 * that overlap on different streams need different workspaces.
 * Replaces the same reference call sites as vx_flash_attn_fwd.
 */
int32_t vx_flash_attn_ws_fwd(const void* q, const void* k, const void* v, void* out, const int32_t* kv_len,
                             const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                             int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                             const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                             const int64_t* out_strides, float scale, void* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * vx_flash_attn_ws_fwd for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation):
 * the same arguments as vx_flash_attn_fwd (calls with a key_bias do not
 * split, as in vx_flash_attn_ws_fwd), and the key split's partials
 * go to a static device array of the library (36 MiB per device, held
 * until the process ends) instead of a workspace. The call allocates
 * nothing. A shape whose split needs more than that scratch fails with
 * VX_ERR_UNSUPPORTED (no MI355X shape does: the plan uses at most 33 MiB).
 * Calls on one device share the scratch: calls that overlap on one device
 * (different streams, or host threads) race and must be serialised by the
 * caller. No counterpart in the reference: it exists for the callers above.
 */
int32_t vx_flash_attn_noalloc_fwd(const void* q, const void* k, const void* v, void* out, const int32_t* kv_len,
                                  const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                                  int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                                  const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* out_strides, float scale, void* stream);

/*
 * Workspace bytes vx_flash_attn_ws_fwd uses for this shape on the current
 * device (0 when it does not split, or on failure). Head dim 64 or 128.
 */
int64_t vx_flash_attn_workspace_size(int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads,
                                     int32_t head_dim);

/*
 * The key-split plan of vx_flash_attn_ws_fwd for a device with num_cus
 * compute units (host only, no GPU): the number of query-tile items split
 * in two, the first key of the second half, and the workspace bytes.
 */
int32_t vx_flash_attn_split_plan(int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                                 int32_t num_cus, int32_t* split_items, int32_t* split_key,
                                 int64_t* workspace_bytes);

/*
 * vx_flash_attn_fwd plus an additive fp32 bias that depends on the head and
 * the query as well as the key (T5's relative-position bias, causal or other
 * boolean masks turned into 0 / -inf):
 *   logit[b, h, i, j] = scale * q.k + bias[b*bs[0] + h*bs[1] + i*bs[2] + j]
 *                       (+ the key-only masks, which may be given as well)
 * bias_strides {batch, head, query} in elements, non-negative multiples of 4
 * (0 broadcasts, e.g. T5's (1, H, L, L) bias over the batch); keys are
 * contiguous and every query row must be readable for round_up(seq_k, 64)
 * elements; bias 16-byte aligned. The bias is read per query row from global
 * memory, which suits the short sequences that use it (text encoders); these
 * calls always run 128-query workgroups (VIDAX_FLASH_BLOCK_SIZES does not
 * apply to them).
 *
 * Replaces the reference's non-kernel branch of dot_product_attention for a
 * head- or query-dependent bias or boolean mask:
 *   - src/vidax/core/attention.py:519-533 (jax.nn.dot_product_attention fallback)
 *   - src/vidax/models/wan/common/t5.py:40-68 (relative-position bias, scale 1)
 *   - src/vidax/models/cosmos3/dit_layers.py:114-116 (causal text pathway)
 */
int32_t vx_flash_attn_bias_fwd(const void* q, const void* k, const void* v, void* out, const int32_t* kv_len,
                               const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                               const float* bias, const int64_t* bias_strides, int32_t batch, int32_t seq_q,
                               int32_t seq_k, int32_t num_heads, int32_t head_dim, const int64_t* q_strides,
                               const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                               float scale, void* stream);

/* Host-only argument check for vx_flash_attn_bias_fwd (no GPU needed). */
int32_t vx_flash_attn_bias_check(const void* q, const void* k, const void* v, const void* out, const int32_t* kv_len,
                                 const uint8_t* key_valid, const float* key_bias, int64_t key_mask_stride,
                                 const float* bias, const int64_t* bias_strides, int32_t batch, int32_t seq_q,
                                 int32_t seq_k, int32_t num_heads, int32_t head_dim, const int64_t* q_strides,
                                 const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                                 float scale);

/*
 * Host-only argument check for vx_flash_attn_fwd (no GPU needed): returns what
 * vx_flash_attn_fwd would return for these arguments before launching.
 * Pointers are checked for NULL-ness and alignment only.
 */
int32_t vx_flash_attn_check(const void* q, const void* k, const void* v, const void* out,
                            const int32_t* kv_len, const uint8_t* key_valid,
                            const float* key_bias, int64_t key_mask_stride,
                            int32_t batch, int32_t seq_q,
                            int32_t seq_k, int32_t num_heads, int32_t head_dim,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* out_strides,
                            float scale);

/*
 * 3D neighbourhood attention forward (NATTEN semantics, boundary-clamped):
 * for query (t, y, x) the window on each axis is [s, s + K') with
 * K' = min(K, L) and s = clamp(i - K'/2, 0, L - K'), so every query sees
 * exactly kt'*kh'*kw' keys and no masking is needed.
 *   out[b,t,y,x,n,:] = sum_{key in window} softmax(scale * q . k) v
 * Logits and softmax statistics in fp32; bf16 in and out.
 *
 * Replaces src/vidax/models/ltx2_5/diffusion_vae.py:179-234
 * (neighborhood_attention_3d, whose caller pre-scales q at :265 -- pass
 * scale = 1.0 for the reference's convention) with window starts as in
 * diffusion_vae.py:152-164 (_window_start).
 *
 * Tensors are contiguous (B, T, Hs, W, NH, D) bf16, 16-byte aligned.
 * Supported: head_dim 128 or 64 (the LTX-2.5 diffusion VAE's,
 * src/vidax/models/ltx2_5/configs.py:194-203), any window (kt, kh, kw >= 1;
 * windows wider than the grid are clamped to it); all sizes >= 1; batch,
 * num_heads <= 65535; w * num_heads * head_dim < 2^30 (one row of tokens).
 */
int32_t vx_na3d_fwd(const void* q, const void* k, const void* v, void* out, int32_t batch,
                    int32_t t, int32_t h, int32_t w, int32_t num_heads, int32_t head_dim,
                    int32_t kernel_t, int32_t kernel_h, int32_t kernel_w, float scale,
                    void* stream);

/* Host-only argument check for vx_na3d_fwd (no GPU needed). */
int32_t vx_na3d_check(const void* q, const void* k, const void* v, const void* out,
                      int32_t batch, int32_t t, int32_t h, int32_t w, int32_t num_heads,
                      int32_t head_dim, int32_t kernel_t, int32_t kernel_h, int32_t kernel_w,
                      float scale);

/*
 * vx_na3d_fwd with the neighbourhood-attention block's q preparation done by
 * the kernel as it loads each query row (q is read once, as projected):
 *   if q_norm_weight != NULL: per-head RMSNorm over head_dim,
 *                     y = bf16(bf16(q * rsqrt(mean(q^2) + eps)) * bf16(w[d]))
 *                     with fp32 statistics (q_norm_weight fp32[head_dim])
 *   if q_post_scale != 1:  y = bf16(y * bf16(q_post_scale))
 *   if rope_cos != NULL:   adjacent pairs (y[2j], y[2j+1]) rotated by the
 *                     token's (rope_cos[s*rope_stride + j], rope_sin[...]) in
 *                     fp32, rounded to bf16; s = (t*h + y)*w + x
 * then out = neighbourhood attention of (y, k, v) with logit scale 1, as
 * vx_na3d_fwd. The rounding points are vx_rmsnorm_scale_rope_fwd's (with
 * per_head_norm = 1); k and v are passed as the block prepares them (k
 * normed and rotated by vx_rmsnorm_scale_rope_fwd). Tables as for that
 * call: fp32, 16-byte aligned, rope_stride a multiple of 4 and >= head_dim/2.
 * Limits and layouts otherwise those of vx_na3d_fwd.
 *
 * Replaces the q half of src/vidax/models/ltx2_5/diffusion_vae.py:263-277
 * (q_norm, q * head_dim**-0.5, _apply_abs_rope(q, ...), then
 * neighborhood_attention_3d), with the tables of _rope_inv_freqs /
 * _default_rope_dim_split (:96-109).
 */
int32_t vx_na3d_qprep_fwd(const void* q, const void* k, const void* v, void* out, int32_t batch, int32_t t,
                          int32_t h, int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t,
                          int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight, float eps,
                          float q_post_scale, const float* rope_cos, const float* rope_sin, int64_t rope_stride,
                          void* stream);

/* Host-only argument check for vx_na3d_qprep_fwd (no GPU needed). */
int32_t vx_na3d_qprep_check(const void* q, const void* k, const void* v, const void* out, int32_t batch, int32_t t,
                            int32_t h, int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t,
                            int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight, float eps,
                            float q_post_scale, const float* rope_cos, const float* rope_sin,
                            int64_t rope_stride);

/*
 * vx_na3d_qprep_fwd with the rotation taken from per-axis rows, as the
 * reference forms it (_apply_abs_rope_axis per t, h and w chunk). rope_cos
 * and rope_sin each hold t + h + w rows of rope_stride floats: rows 0..t-1
 * the t axis, rows t..t+h-1 the h axis, rows t+h..t+h+w-1 the w axis, each
 * row's value for pair j at column j. With rope_split = (d_t, d_h, d_w), pair
 * j of token (tt, y, x) turns by
 *   (rope_cos[tt*rope_stride + j], rope_sin[...])            j < d_t/2
 *   (rope_cos[(t + y)*rope_stride + j], ...)                 j < (d_t+d_h)/2
 *   (rope_cos[(t + h + x)*rope_stride + j], ...)             otherwise
 * which equals vx_na3d_qprep_fwd with the per-token tables that concatenate
 * these parts (create_abs_rope3d_freqs's), bit for bit. Tables fp32, 16-byte
 * aligned, rope_stride a multiple of 4 and >= head_dim/2, (t+h+w)*rope_stride
 * < 2^31; d_t, d_h, d_w even and summing to head_dim, d_t and d_h multiples
 * of 8 (the default split of head dims 64 and 128 is). rope_split = NULL: no
 * rotation. A few hundred rows replace one table row per token, which every
 * head's workgroups re-read.
 *
 * Replaces the q half of src/vidax/models/ltx2_5/diffusion_vae.py:263-277
 * with _apply_abs_rope's per-axis tables (:112-149, _rope_inv_freqs :106-109).
 */
int32_t vx_na3d_qprep_axes_fwd(const void* q, const void* k, const void* v, void* out, int32_t batch, int32_t t,
                               int32_t h, int32_t w, int32_t num_heads, int32_t head_dim, int32_t kernel_t,
                               int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight, float eps,
                               float q_post_scale, const float* rope_cos, const float* rope_sin, int64_t rope_stride,
                               const int32_t* rope_split, void* stream);

/* Host-only argument check for vx_na3d_qprep_axes_fwd (no GPU needed). */
int32_t vx_na3d_qprep_axes_check(const void* q, const void* k, const void* v, const void* out, int32_t batch,
                                 int32_t t, int32_t h, int32_t w, int32_t num_heads, int32_t head_dim,
                                 int32_t kernel_t, int32_t kernel_h, int32_t kernel_w, const float* q_norm_weight,
                                 float eps, float q_post_scale, const float* rope_cos, const float* rope_sin,
                                 int64_t rope_stride, const int32_t* rope_split);

/*
 * Fused attention prologue: RMSNorm and/or 3D rotary embedding of q or k in
 * one pass (read x once, write out once), bf16 in and out. For each token row
 * (num_heads * head_dim values, contiguous):
 *   if weight != NULL:  y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * bf16(weight))
 *                       with the mean over the whole row (per_head_norm = 0,
 *                       Wan's q/k norm over the projected dim) or over each
 *                       head (per_head_norm = 1); fp32 statistics; weight is
 *                       fp32[num_heads * head_dim]
 *   else                y = x
 *   if rope_cos != NULL: every head's adjacent pairs (y[2j], y[2j+1]) are
 *                       rotated by (rope_cos[s*rope_stride + j],
 *                       rope_sin[s*rope_stride + j]) in fp32 and rounded to bf16
 * Output rows have the same (B, S, H, D) layout as the input.
 *
 * Replaces the reference's q/k prologue of the DiT attention:
 *   - src/vidax/core/attention.py:149-161 (RMSNorm: fp32 normalise, cast,
 *     times the cast scale)
 *   - src/vidax/core/rope3d.py:88-111 (apply_rope3d: adjacent-pair rotation in
 *     fp32, cast back), with tables from rope3d.py:45-86 (create_rope3d_freqs)
 *   - their use in src/vidax/models/wan/common/dit_layers.py:135-149
 *
 * Strides {batch, seq} are in elements (NULL = contiguous rows of
 * num_heads * head_dim), non-negative multiples of 8; x, out, weight and the
 * tables 16-byte aligned; rope_stride a multiple of 4, >= head_dim / 2.
 * out may equal x (in place) when the strides are the same.
 * Supported: head_dim 64 or 128, num_heads * head_dim <= 8192.
 */
int32_t vx_rmsnorm_rope_fwd(const void* x, void* out, const float* weight, float eps, int32_t per_head_norm,
                            const float* rope_cos, const float* rope_sin, int64_t rope_stride, int32_t batch,
                            int32_t seq, int32_t num_heads, int32_t head_dim, const int64_t* x_strides,
                            const int64_t* out_strides, void* stream);

/* Host-only argument check for vx_rmsnorm_rope_fwd (no GPU needed). */
int32_t vx_rmsnorm_rope_check(const void* x, const void* out, const float* weight, float eps, int32_t per_head_norm,
                              const float* rope_cos, const float* rope_sin, int64_t rope_stride, int32_t batch,
                              int32_t seq, int32_t num_heads, int32_t head_dim, const int64_t* x_strides,
                              const int64_t* out_strides);

/*
 * vx_rmsnorm_rope_fwd with one more step between the norm and the rotation:
 *   if post_scale != 1:  y = bf16(y * bf16(post_scale))
 * (vx_rmsnorm_rope_fwd is this call with post_scale = 1). post_scale must be
 * finite; all other arguments and limits are vx_rmsnorm_rope_fwd's.
 *
 * Replaces the q/k preparation of the LTX-2.5 diffusion-VAE neighbourhood
 * attention block, src/vidax/models/ltx2_5/diffusion_vae.py:255-273: per-head
 * RMSNorm (q_norm / k_norm, per_head_norm = 1), q * head_dim^-0.5 (a bf16
 * array times a weakly typed scalar: the scalar is rounded to bf16), then the
 * absolute interleaved-pair RoPE of _apply_abs_rope (:106-149) with per-token
 * tables of the (T, H, W) split of _default_rope_dim_split (:96-103). The
 * rows are the (B, T, H, W, NH, HD) tokens, seq = T * H * W.
 */
int32_t vx_rmsnorm_scale_rope_fwd(const void* x, void* out, const float* weight, float eps, int32_t per_head_norm,
                                  float post_scale, const float* rope_cos, const float* rope_sin,
                                  int64_t rope_stride, int32_t batch, int32_t seq, int32_t num_heads,
                                  int32_t head_dim, const int64_t* x_strides, const int64_t* out_strides,
                                  void* stream);

/* Host-only argument check for vx_rmsnorm_scale_rope_fwd (no GPU needed). */
int32_t vx_rmsnorm_scale_rope_check(const void* x, const void* out, const float* weight, float eps,
                                    int32_t per_head_norm, float post_scale, const float* rope_cos,
                                    const float* rope_sin, int64_t rope_stride, int32_t batch, int32_t seq,
                                    int32_t num_heads, int32_t head_dim, const int64_t* x_strides,
                                    const int64_t* out_strides);

/*
 * Launch plan of vx_flash_attn_fwd / vx_flash_attn_bias_fwd for a shape (host
 * only, no GPU): writes the name of the kernel those calls would launch,
 * "flash_fwd_kernel<mask_kind, head_dim, waves>" or
 * "flash_stream_kernel<head_dim>", into kernel_name (name_len bytes,
 * NUL-terminated). mask_kind is a bit set: 1 key_valid, 2 key_bias, 4 a
 * per-(query, key) bias. waves is 8 (256-query workgroups) for long key
 * sequences on large grids, else 4 (128-query workgroups), per the
 * library's gfx950 tile table; key sequences up to 1024 with no key masks
 * but kv_len, at most 64 batch items and at least 4096 256-query tiles (up
 * to about 500k tile-steps) run the persistent 256-query kernel
 * flash_stream_kernel (one workgroup per CU; on a device with fewer than 256
 * CUs a grid too large for its item table runs the 4-wave kernel instead).
 * The environment variable
 * VIDAX_FLASH_BLOCK_SIZES="block_q,block_k_major,block_k" (block_q 128 or
 * 256, key tiles 64) or "default" overrides the workgroup size (128 turns the
 * persistent kernel off). A per-(query, key) bias, or key_valid together
 * with key_bias, always runs 4 waves. The variable is read once,
 * at the first flash call or plan of the process; a malformed value makes
 * every flash call and plan fail with VX_ERR_INVALID_ARGUMENT, an
 * unsupported one with VX_ERR_UNSUPPORTED.
 *
 * Replaces the reference's tile-size selection:
 *   - src/vidax/core/attention.py:10-35 (_FLASH_BLOCK_SIZES_BY_DEVICE_KIND,
 *     _flash_block_sizes and its VIDAX_FLASH_BLOCK_SIZES override)
 */
int32_t vx_flash_attn_plan(int32_t batch, int32_t seq_q, int32_t seq_k, int32_t num_heads, int32_t head_dim,
                           int32_t mask_kind, char* kernel_name, int32_t name_len);

/*
 * Launch plan of vx_na3d_fwd (host only): the name of the kernel chosen by
 * the clamped x window (at head dim 64 also by the grid's h and w, which
 * decide the brick shape; and by the clamped t window min(kernel_t, t), which
 * decides the brick depth), e.g. "na3d_tstack_kernel<128>", written as by
 * vx_flash_attn_plan. Fails as vx_na3d_check would for the same sizes.
 * Part of the replacement of src/vidax/models/ltx2_5/diffusion_vae.py:179-234.
 */
int32_t vx_na3d_plan(int32_t t, int32_t h, int32_t w, int32_t head_dim, int32_t kernel_t, int32_t kernel_h,
                     int32_t kernel_w, char* kernel_name, int32_t name_len);

/*
 * Name of the kernel launched by the last successful vx_*_fwd call on the
 * calling thread ("" before the first), recorded by the launcher from the
 * launched instantiation. For tests and profiling: it observes the launch
 * itself rather than a copy of the launch rule.
 */
const char* vx_last_launch(void);

/*
 * Failure injection for error-path tests: while `code` is non-zero, every
 * vx_*_fwd call that passes argument checks returns `code` without launching,
 * with a message naming the injection. 0 turns it off. Process-wide.
 */
void vx_debug_inject_error(int32_t code);

/*
 * Measurement hook (no counterpart in the reference; not part of the
 * attention path): launches n_groups (1..4096) one-wave workgroups on
 * `stream`, each storing four uint64 at out[4*g]: the XCD it ran on, its
 * hardware id (HW_REG_HW_ID: shader engine, CU, SIMD, wave slot), the
 * shader clock counter (read per CU) and the real-time counter, read when it
 * runs. *wall_clock_khz receives the real-time counter's rate. Two stamps
 * around a run of kernels on one stream give, per CU found in both, the
 * shader cycles and the wall time that passed: the clock the chip held
 * under that load. `out` is device memory, 8-byte aligned, of 4 * n_groups
 * uint64.
 */
int32_t vx_debug_clock_stamp(uint64_t* out, int32_t n_groups, int32_t* wall_clock_khz, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VX_ATTN_H_ */
