"""vidax_amd: MI355X (gfx950) HIP kernels for vidax's DiT attention hot path.

Drop-in replacements for the reference's attention entry points:
  dot_product_attention, local_attention   (src/vidax/core/attention.py)
  masked_self_attention                   (src/vidax/models/hunyuan_video/common/dit_layers.py)
  neighborhood_attention_3d               (src/vidax/models/ltx2_5/diffusion_vae.py)
and the q/k prologue in front of them:
  rms_norm, create_rope3d_freqs, apply_rope3d, qk_norm_rope
                                          (src/vidax/core/attention.py, rope3d.py)
  default_rope_dim_split, create_abs_rope3d_freqs, create_abs_rope3d_axis_freqs,
  apply_abs_rope3d, na3d_qk_norm_rope     (src/vidax/models/ltx2_5/diffusion_vae.py)
all backed by libvx_attn.so (C ABI: include/vx_attn.h).
"""
from .attention import (dot_product_attention, flash_attention, flash_supported, local_attention,
                        masked_self_attention)
from .natten import na3d_block_attention, neighborhood_attention_3d
from .prologue import (AbsRope3dAxes, apply_abs_rope3d, apply_rope3d, create_abs_rope3d_axis_freqs,
                       create_abs_rope3d_freqs, create_rope3d_freqs, default_rope_dim_split, na3d_qk_norm_rope,
                       qk_norm_rope, rms_norm)

__all__ = [
    "dot_product_attention",
    "flash_attention",
    "flash_supported",
    "local_attention",
    "masked_self_attention",
    "neighborhood_attention_3d",
    "na3d_block_attention",
    "rms_norm",
    "create_rope3d_freqs",
    "apply_rope3d",
    "qk_norm_rope",
    "default_rope_dim_split",
    "create_abs_rope3d_freqs",
    "create_abs_rope3d_axis_freqs",
    "AbsRope3dAxes",
    "apply_abs_rope3d",
    "na3d_qk_norm_rope",
]
