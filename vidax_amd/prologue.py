"""Attention prologue: RMSNorm of q/k and the 3D rotary embedding, on the GPU.

Mirrors the reference's q/k preparation in the DiT attention block:
`RMSNorm` (`src/vidax/core/attention.py:149-161`), `create_rope3d_freqs` and
`apply_rope3d` (`src/vidax/core/rope3d.py:45-111`), as used by Wan's `attend`
(`src/vidax/models/wan/common/dit_layers.py:135-149`), and the LTX-2.5
diffusion-VAE neighbourhood block's per-head norm, q scaling and absolute
RoPE (`src/vidax/models/ltx2_5/diffusion_vae.py:96-149,255-273`). The norm,
the scaling and the rotation run in one HIP kernel
(`vx_rmsnorm_scale_rope_fwd`) that reads each bf16 row once and writes it
once; `qk_norm_rope` and `na3d_qk_norm_rope` are the fused forms of the
reference's norm -> (scale) -> rope sequences.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional, Tuple

import torch

from . import _lib

__all__ = ["create_rope3d_freqs", "apply_rope3d", "rms_norm", "qk_norm_rope",
           "default_rope_dim_split", "create_abs_rope3d_freqs", "create_abs_rope3d_axis_freqs", "AbsRope3dAxes",
           "apply_abs_rope3d", "na3d_qk_norm_rope"]


def _axis_freqs(seq_len: int, dim: int, theta: float, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) of shape (seq_len, dim // 2), fp32 (`rope3d.py:34-42`)."""
    inv_freq = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float32, device=device),
                               torch.arange(0, dim, 2, dtype=torch.float32, device=device) / dim)
    angles = torch.outer(torch.arange(seq_len, dtype=torch.float32, device=device), inv_freq)
    return torch.cos(angles), torch.sin(angles)


def create_rope3d_freqs(t: int, h: int, w: int, head_dim: int, theta: float = 10000.0,
                        max_seq_len: int = 1024, device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-position rotation tables for a (t, h, w) grid: (cos, sin), each
    (1, t*h*w, 1, head_dim // 2) fp32, with the head_dim // 2 frequency pairs
    split c - 2*(c//3) / c//3 / c//3 over the T / H / W axes
    (`rope3d.py:45-86`)."""
    if head_dim % 2:
        raise ValueError("head_dim must be even")
    c = head_dim // 2
    dim_t, dim_h, dim_w = c - 2 * (c // 3), c // 3, c // 3
    ct, st = _axis_freqs(max_seq_len, 2 * dim_t, theta, device)
    ch, sh = _axis_freqs(max_seq_len, 2 * dim_h, theta, device)
    cw, sw = _axis_freqs(max_seq_len, 2 * dim_w, theta, device)

    def grid(ft, fh, fw):
        gt = ft[:t, None, None, :].expand(t, h, w, dim_t)
        gh = fh[None, :h, None, :].expand(t, h, w, dim_h)
        gw = fw[None, None, :w, :].expand(t, h, w, dim_w)
        return torch.cat([gt, gh, gw], dim=-1).reshape(t * h * w, c)

    return grid(ct, ch, cw)[None, :, None, :], grid(st, sh, sw)[None, :, None, :]


def _check_x(x: torch.Tensor, name: str = "x") -> None:
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16; got {x.dtype}")
    if not x.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")


def _tables(freqs, seq: int, half: int, device) -> Tuple[torch.Tensor, torch.Tensor, int]:
    cos, sin = freqs
    cos = torch.as_tensor(cos, device=device).to(torch.float32).reshape(-1, half)
    sin = torch.as_tensor(sin, device=device).to(torch.float32).reshape(-1, half)
    if cos.shape[0] != seq or sin.shape[0] != seq:
        raise ValueError(f"rope tables hold {cos.shape[0]} positions, the sequence has {seq}")
    stride = (half + 3) // 4 * 4
    if stride != half:
        cos = torch.nn.functional.pad(cos, (0, stride - half))
        sin = torch.nn.functional.pad(sin, (0, stride - half))
    return cos.contiguous(), sin.contiguous(), stride


def _run(x4: torch.Tensor, out4: torch.Tensor, weight: Optional[torch.Tensor], eps: float, per_head: bool,
         tables, post_scale: float = 1.0) -> None:
    B, S, H, D = x4.shape
    if x4.stride(3) != 1 or x4.stride(2) != D:
        raise ValueError("each token row (num_heads * head_dim) must be contiguous")
    cos_t = sin_t = None
    stride = 0
    if tables is not None:
        cos_t, sin_t, stride = tables
    xs = _lib.strides2((x4.stride(0), x4.stride(1)))
    os_ = _lib.strides2((out4.stride(0), out4.stride(1)))
    stream = torch.cuda.current_stream(x4.device).cuda_stream
    with torch.cuda.device(x4.device):
        rc = _lib.lib().vx_rmsnorm_scale_rope_fwd(
            x4.data_ptr(), out4.data_ptr(),
            weight.data_ptr() if weight is not None else None, ctypes.c_float(eps), int(per_head),
            ctypes.c_float(post_scale), cos_t.data_ptr() if cos_t is not None else None, sin_t.data_ptr() if sin_t is not None else None,
            stride, B, S, H, D, xs, os_, ctypes.c_void_p(stream))
    _lib.raise_for(rc)


def _head_dim_for(length: int) -> int:
    for d in (128, 64):
        if length % d == 0:
            return d
    raise NotImplementedError(f"rows of length {length} are not a multiple of 64")


def apply_rope3d(x: torch.Tensor, freqs) -> torch.Tensor:
    """Rotates adjacent (even, odd) pairs of every head of x (B, S, H, D) by
    the per-position (cos, sin) of `freqs` (broadcastable to (1, S, 1, D//2)),
    in fp32, returning bf16 (`rope3d.py:88-111`)."""
    _check_x(x)
    if x.dim() != 4:
        raise ValueError("x must be (B, S, num_heads, head_dim)")
    x = x.contiguous()
    out = torch.empty_like(x)
    _run(x, out, None, 0.0, False, _tables(freqs, x.shape[1], x.shape[3] // 2, x.device))
    return out


def rms_norm(x: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last axis: bf16(bf16(x * rsqrt(mean(x^2) + eps)) *
    bf16(scale)) with fp32 statistics (`attention.py:149-161`). x is
    (..., L) bf16 with L a multiple of 64 (the projected q/k) or (B, S, H, D)
    with the norm over each head's D."""
    _check_x(x)
    scale = torch.as_tensor(scale, device=x.device).to(torch.float32).reshape(-1)
    L = x.shape[-1]
    if scale.numel() != L:
        raise ValueError(f"scale has {scale.numel()} entries, x's last axis {L}")
    if x.dim() == 4:
        B, S, H, D = x.shape
        x4 = x.contiguous()
        weight = scale.repeat(H).contiguous()
        per_head = True
    else:
        lead = x.shape[:-1]
        D = _head_dim_for(L)
        x4 = x.contiguous().reshape(1, -1, L // D, D)
        weight = scale.contiguous()
        per_head = False
    out4 = torch.empty_like(x4)
    _run(x4, out4, weight, float(eps), per_head, None)
    return out4.reshape(x.shape)


def qk_norm_rope(x: torch.Tensor, scale: Optional[torch.Tensor], freqs, num_heads: int,
                 eps: float = 1e-6) -> torch.Tensor:
    """Fused Wan q/k prologue (`dit_layers.py:135-149`): x (B, S, num_heads *
    head_dim) bf16 -> RMSNorm over the whole projected row (skipped when
    scale is None) -> reshape to (B, S, num_heads, head_dim) -> apply_rope3d
    with `freqs` (skipped when None), in one pass."""
    _check_x(x)
    if x.dim() != 3:
        raise ValueError("x must be (B, S, num_heads * head_dim)")
    B, S, L = x.shape
    if L % num_heads:
        raise ValueError(f"row length {L} is not divisible by num_heads {num_heads}")
    D = L // num_heads
    x4 = x.reshape(B, S, num_heads, D) if x.stride(2) == 1 else x.contiguous().reshape(B, S, num_heads, D)
    out4 = torch.empty((B, S, num_heads, D), dtype=x.dtype, device=x.device)
    weight = None
    if scale is not None:
        weight = torch.as_tensor(scale, device=x.device).to(torch.float32).reshape(-1).contiguous()
        if weight.numel() != L:
            raise ValueError(f"scale has {weight.numel()} entries, rows have {L}")
    tables = _tables(freqs, S, D // 2, x.device) if freqs is not None else None
    _run(x4, out4, weight, float(eps), False, tables)
    return out4


# ------------------------------------------------ neighbourhood-attention block
def default_rope_dim_split(head_dim: int) -> Tuple[int, int, int]:
    """(d_t, d_h, d_w) channels of head_dim given to the T, H and W rotations:
    d_t = (head_dim // 4) rounded down to even, the rest halved, d_t lowered
    by 2 when that half is odd (`diffusion_vae.py:96-103`)."""
    d_t = (head_dim // 4) // 2 * 2
    d_hw = (head_dim - d_t) // 2
    if d_hw % 2:
        d_t -= 2
        d_hw = (head_dim - d_t) // 2
    return d_t, d_hw, d_hw


def _abs_rope_split(head_dim: int, rope_split) -> Tuple[int, int, int]:
    d_t, d_h, d_w = rope_split or default_rope_dim_split(head_dim)
    if d_t + d_h + d_w != head_dim or d_t % 2 or d_h % 2 or d_w % 2:
        raise ValueError(f"rope split {(d_t, d_h, d_w)} must be even and sum to head_dim {head_dim}")
    return d_t, d_h, d_w


def _abs_rope_axis(n: int, d: int, base: float, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos and sin (n, d/2) of positions 0..n-1 times one axis's inverse
    frequencies 1 / base^(arange(0, d, 2) / d), the frequencies computed in
    float64 and stored as fp32, the angles formed in fp32
    (`diffusion_vae.py:106-128`)."""
    inv = 1.0 / torch.pow(torch.tensor(float(base), dtype=torch.float64),
                          torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = torch.arange(n, dtype=torch.float32, device=device)[:, None] * inv.to(torch.float32).to(device)[None, :]
    return torch.cos(ang), torch.sin(ang)


class AbsRope3dAxes(NamedTuple):
    """Per-axis rows of the absolute interleaved-pair RoPE of a (t, h, w) grid:
    cos and sin, each (t + h + w, stride) fp32 (stride = head_dim/2 rounded up
    to 4 floats): rows 0..t-1 hold the t axis's angles in the t pairs'
    columns, the next h rows the h axis's in the h columns, the last w rows
    the w axis's in the w columns (other columns zero); `grid` = (t, h, w),
    `split` = (d_t, d_h, d_w)."""
    cos: torch.Tensor
    sin: torch.Tensor
    grid: Tuple[int, int, int]
    split: Tuple[int, int, int]


def create_abs_rope3d_axis_freqs(t: int, h: int, w: int, head_dim: int,
                                 rope_split: Optional[Tuple[int, int, int]] = None, base: float = 10000.0,
                                 device=None) -> AbsRope3dAxes:
    """The per-axis form of create_abs_rope3d_freqs, as the reference builds
    it (`diffusion_vae.py:112-128`, `_apply_abs_rope_axis` per chunk): the t,
    h and w rows of the same values that create_abs_rope3d_freqs concatenates
    per token, in one table. For na3d_block_attention, whose kernel then reads
    a few hundred rows instead of one table row per token and head."""
    split = _abs_rope_split(head_dim, rope_split)
    width = -(-(head_dim // 2) // 4) * 4
    cos = torch.zeros((t + h + w, width), dtype=torch.float32, device=device)
    sin = torch.zeros_like(cos)
    row, col = 0, 0
    for n, d in zip((t, h, w), split):
        c, s_ = _abs_rope_axis(n, d, base, device)
        cos[row:row + n, col:col + d // 2] = c
        sin[row:row + n, col:col + d // 2] = s_
        row += n
        col += d // 2
    return AbsRope3dAxes(cos, sin, (t, h, w), tuple(split))


def create_abs_rope3d_freqs(t: int, h: int, w: int, head_dim: int,
                            rope_split: Optional[Tuple[int, int, int]] = None, base: float = 10000.0,
                            device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-token tables of the absolute interleaved-pair RoPE of a (t, h, w)
    grid: (cos, sin), each (1, t*h*w, 1, head_dim // 2) fp32. Pair j < d_t/2
    turns by t_pos * inv_t[j], the next d_h/2 pairs by h_pos * inv_h, the last
    d_w/2 by w_pos * inv_w, with inv = 1 / base^(arange(0, d, 2) / d) computed
    in float64 and stored as fp32 and the angles formed in fp32
    (`diffusion_vae.py:106-149,265-273`)."""
    d_t, d_h, d_w = _abs_rope_split(head_dim, rope_split)
    (ct, st), (ch, sh), (cw, sw) = (_abs_rope_axis(n, d, base, device) for n, d in ((t, d_t), (h, d_h), (w, d_w)))

    def grid(ft, fh, fw):
        gt = ft[:, None, None, :].expand(t, h, w, d_t // 2)
        gh = fh[None, :, None, :].expand(t, h, w, d_h // 2)
        gw = fw[None, None, :, :].expand(t, h, w, d_w // 2)
        return torch.cat([gt, gh, gw], dim=-1).reshape(1, t * h * w, 1, head_dim // 2)

    return grid(ct, ch, cw), grid(st, sh, sw)


def _check_grid(x: torch.Tensor) -> None:
    _check_x(x)
    if x.dim() != 6:
        raise ValueError("x must be (B, T, H, W, num_heads, head_dim)")


def apply_abs_rope3d(x: torch.Tensor, freqs) -> torch.Tensor:
    """`_apply_abs_rope` (`diffusion_vae.py:130-149`) of x (B, T, H, W, NH,
    HD) with tables from create_abs_rope3d_freqs: fp32 rotation of each
    head's (even, odd) pairs, cast back to bf16."""
    _check_grid(x)
    B, T, H, W, NH, HD = x.shape
    x4 = x.contiguous().reshape(B, T * H * W, NH, HD)
    out4 = torch.empty_like(x4)
    _run(x4, out4, None, 0.0, False, _tables(freqs, T * H * W, HD // 2, x.device))
    return out4.reshape(x.shape)


def na3d_qk_norm_rope(x: torch.Tensor, scale: Optional[torch.Tensor], freqs, eps: float = 1e-6,
                      post_scale: float = 1.0) -> torch.Tensor:
    """The q/k preparation of the neighbourhood-attention block in one pass
    (`diffusion_vae.py:263-273`): per-head RMSNorm with weight `scale`
    (head_dim,) (skipped when None), times `post_scale` as a bf16 scalar (q:
    head_dim ** -0.5; k: 1.0), then the absolute RoPE with `freqs` from
    create_abs_rope3d_freqs (skipped when None). x is (B, T, H, W, NH, HD)
    bf16; the result has the same shape."""
    _check_grid(x)
    B, T, H, W, NH, HD = x.shape
    x4 = x.contiguous().reshape(B, T * H * W, NH, HD)
    out4 = torch.empty_like(x4)
    weight = None
    if scale is not None:
        w = torch.as_tensor(scale, device=x.device).to(torch.float32).reshape(-1)
        if w.numel() != HD:
            raise ValueError(f"scale has {w.numel()} entries, head_dim is {HD}")
        weight = w.repeat(NH).contiguous()
    tables = _tables(freqs, T * H * W, HD // 2, x.device) if freqs is not None else None
    _run(x4, out4, weight, float(eps), True, tables, float(post_scale))
    return out4.reshape(x.shape)
