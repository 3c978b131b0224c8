"""3D neighbourhood attention entry point over the gfx950 HIP kernel.

Mirrors `neighborhood_attention_3d(q, k, v, kernel_size)` of
`src/vidax/models/ltx2_5/diffusion_vae.py:179-234`: (B, T, H, W, NH, HD)
tensors, q already pre-scaled by the caller (`diffusion_vae.py:265`), NATTEN
boundary-clamped windows (`diffusion_vae.py:152-164`), output of the same shape.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

__all__ = ["neighborhood_attention_3d", "na3d_attention", "na3d_kernel_name", "na3d_block_attention"]


def na3d_kernel_name(width: int, kernel_w: int, head_dim: int = 128, height: Optional[int] = None,
                     depth: int = 1, kernel_t: int = 1) -> str:
    """Name of the kernel the library launches for this x window (the C ABI's
    launch plan): row streaming with 16-key x segments up to kw' = 9 (at head
    dim 64 the tall bricks instead when they pad the height x width plane no
    more; at head dim 128 bricks of two t planes when kt' >= 2), its
    tall-brick form up to kw' = 13 (at head dim 64 in 32-wide
    bricks when the width rounds up to the same multiple of 16 and 32, two t
    planes deep for t windows kt' = min(kernel_t, depth) of 5 and more),
    32-key segments up to kw' = 25, the per-wave kernel above that
    (kw' = min(kw, W)). The grid height decides the choice at head dim 64
    with kw' <= 9 and must be given there; depth (the grid's t extent) and
    kernel_t matter at head dim 128 with kw' <= 9 and at head dim 64 with
    9 < kw' <= 13."""
    kw_c = min(int(kernel_w), int(width))
    if height is None:
        if int(head_dim) == 64 and kw_c <= 9:
            raise ValueError("na3d_kernel_name: at head_dim 64 with an x window of at most 9 the kernel "
                             "depends on the grid height; pass height=")
        height = 1
    return _lib.na3d_plan(int(depth), int(height), int(width), int(head_dim), int(kernel_t), 1, int(kernel_w))


def _pad_rows(t: torch.Tensor) -> torch.Tensor:
    """A copy of a 2-D fp32 table whose rows are padded to a multiple of 4
    floats (16-byte aligned rows)."""
    width = -(-t.shape[1] // 4) * 4
    out = torch.zeros((t.shape[0], width), dtype=torch.float32, device=t.device)
    out[:, :t.shape[1]] = t
    return out


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def na3d_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   kernel_size: Tuple[int, int, int], scale: float = 1.0,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Neighbourhood attention with an explicit logit scale (1.0 = reference)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.dim() != 6:
            raise ValueError(f"{name} must be (B, T, H, W, NH, HD); got {tuple(t.shape)}")
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16; got {t.dtype}")
        if not t.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k and v must have the same shape")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k and v must be on the same device")
    if len(kernel_size) != 3:
        raise ValueError("kernel_size must be (kt, kh, kw)")
    # the kernel reads 16-byte chunks: contiguous tensors at 16-byte aligned
    # addresses (a contiguous view at an odd offset is copied)
    q, k, v = (_aligned16(t) for t in (q, k, v))
    B, T, H, W, NH, HD = q.shape
    if out is None:
        out = torch.empty_like(q)
    elif (out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous() or
          out.device != q.device or out.data_ptr() % 16 != 0):
        raise ValueError("out must be a contiguous, 16-byte aligned bf16 tensor shaped like q, on q's device")
    stream = torch.cuda.current_stream(q.device).cuda_stream
    with torch.cuda.device(q.device):
        rc = _lib.lib().vx_na3d_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            B, T, H, W, NH, HD, int(kernel_size[0]), int(kernel_size[1]), int(kernel_size[2]),
            ctypes.c_float(scale), ctypes.c_void_p(stream))
    _lib.raise_for(rc)
    return out


def neighborhood_attention_3d(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              kernel_size: Tuple[int, int, int]) -> torch.Tensor:
    """NATTEN-semantics 3D neighbourhood attention; q is pre-scaled by the caller."""
    return na3d_attention(q, k, v, kernel_size, scale=1.0)


def na3d_block_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         kernel_size: Tuple[int, int, int], q_norm_weight: Optional[torch.Tensor], freqs,
                         eps: float = 1e-6, q_post_scale: Optional[float] = None,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of the LTX-2.5 neighbourhood-attention block with q prepared
    inside the kernel (`src/vidax/models/ltx2_5/diffusion_vae.py:263-277`):
    q as projected (B, T, H, W, NH, HD) goes through per-head RMSNorm with
    `q_norm_weight` (HD,) (skipped when None), times bf16(q_post_scale)
    (default HD ** -0.5, the block's `q * head_dim ** -0.5`), and the absolute
    RoPE with `freqs` from `create_abs_rope3d_freqs` or, read per axis and
    with the same result, `create_abs_rope3d_axis_freqs` (skipped when None),
    as the kernel loads each query row; k (normed and rotated, e.g. by
    `na3d_qk_norm_rope`) and v are used as given. Equals
    `neighborhood_attention_3d(na3d_qk_norm_rope(q, ...), k, v, kernel_size)`
    without the separate pass over q."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or t.dim() != 6 or t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a (B, T, H, W, NH, HD) bf16 GPU tensor")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k and v must have the same shape")
    if len(kernel_size) != 3:
        raise ValueError("kernel_size must be (kt, kh, kw)")
    q, k, v = (_aligned16(t) for t in (q, k, v))
    B, T, H, W, NH, HD = q.shape
    if q_post_scale is None:
        q_post_scale = HD ** -0.5
    weight = None
    if q_norm_weight is not None:
        weight = torch.as_tensor(q_norm_weight, device=q.device).to(torch.float32).reshape(-1).contiguous()
        if weight.numel() != HD:
            raise ValueError(f"q_norm_weight has {weight.numel()} entries, head_dim is {HD}")
    from .prologue import AbsRope3dAxes
    axes = isinstance(freqs, AbsRope3dAxes)
    cos_t = sin_t = None
    stride = 0
    if freqs is not None and not axes:
        from .prologue import _tables
        cos_t, sin_t, stride = _tables(freqs, T * H * W, HD // 2, q.device)
    if axes:
        # one fp32 table each of T + H + W rows (t axis, h axis, w axis)
        if tuple(freqs.grid) != (T, H, W):
            raise ValueError(f"per-axis rope rows built for the grid {tuple(freqs.grid)}, not {(T, H, W)}")
        for tab in (freqs.cos, freqs.sin):
            if (tab.dim() != 2 or tab.shape[0] != T + H + W or tab.shape[1] < HD // 2
                    or tab.dtype != torch.float32 or tab.device != q.device):
                raise ValueError(f"per-axis rope table {tuple(tab.shape)} is not ({T + H + W}, >= {HD // 2}) "
                                 "fp32 on q's device")
        # rows 16-byte aligned and the same stride in both tables
        ax_c, ax_s = freqs.cos, freqs.sin
        if not (ax_c.stride(1) == 1 and ax_c.stride(0) % 4 == 0 and ax_c.data_ptr() % 16 == 0):
            ax_c = _pad_rows(ax_c)
        if not (ax_s.stride(1) == 1 and ax_s.stride(0) == ax_c.stride(0) and ax_s.data_ptr() % 16 == 0):
            ax_s = _pad_rows(ax_s)
        if ax_s.stride(0) != ax_c.stride(0):
            ax_c = _pad_rows(ax_c)
        ax_split = (ctypes.c_int32 * 3)(*[int(d) for d in freqs.split])
    if out is None:
        out = torch.empty_like(q)
    elif (out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous() or
          out.device != q.device or out.data_ptr() % 16 != 0):
        raise ValueError("out must be a contiguous, 16-byte aligned bf16 tensor shaped like q, on q's device")
    stream = torch.cuda.current_stream(q.device).cuda_stream
    with torch.cuda.device(q.device):
        if axes:
            rc = _lib.lib().vx_na3d_qprep_axes_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                B, T, H, W, NH, HD, int(kernel_size[0]), int(kernel_size[1]), int(kernel_size[2]),
                weight.data_ptr() if weight is not None else None, ctypes.c_float(eps),
                ctypes.c_float(q_post_scale),
                ax_c.data_ptr(), ax_s.data_ptr(), int(ax_c.stride(0)), ax_split, ctypes.c_void_p(stream))
        else:
            rc = _lib.lib().vx_na3d_qprep_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                B, T, H, W, NH, HD, int(kernel_size[0]), int(kernel_size[1]), int(kernel_size[2]),
                weight.data_ptr() if weight is not None else None, ctypes.c_float(eps),
                ctypes.c_float(q_post_scale),
                cos_t.data_ptr() if cos_t is not None else None,
                sin_t.data_ptr() if sin_t is not None else None, stride, ctypes.c_void_p(stream))
    _lib.raise_for(rc)
    return out
