"""CPU oracle of the attention prologue (q/k RMSNorm, 3D rotary embedding) --
test infrastructure only (used by tests/ as the checker).

Restates, in numpy with the reference's dtype points:
  - RMSNorm, `src/vidax/core/attention.py:149-161`: x to fp32, mean of squares
    over the last axis, x * rsqrt(var + eps), cast to bf16, times the scale
    cast to bf16 (a bf16 x bf16 product, exact in fp32, then rounded).
  - create_rope3d_freqs, `src/vidax/core/rope3d.py:34-86`: per-axis
    inv_freq = 1 / theta^(arange(0, dim, 2) / dim) and angles
    pos * inv_freq in fp32, split c - 2*(c//3) / c//3 / c//3 over T/H/W.
  - apply_rope3d, `src/vidax/core/rope3d.py:88-111`: adjacent pairs
    (x[2j], x[2j+1]) -> (x1*cos - x2*sin, x2*cos + x1*sin) in fp32, cast to bf16.
  - the LTX-2.5 diffusion-VAE neighbourhood block's q/k preparation,
    `src/vidax/models/ltx2_5/diffusion_vae.py:96-149,255-273`:
    _default_rope_dim_split, _rope_inv_freqs (float64 exponents, stored
    fp32), per-head RMSNorm, q * head_dim^-0.5 as bf16 x bf16(scalar), and
    _apply_abs_rope: fp32 rotation of the (even, odd) pairs of the T, H and W
    chunks by integer positions times the axis frequencies, cast back.

Parity notes: the mean of squares and rsqrt are fp32 operations whose last
bit depends on summation order and on the rsqrt implementation (XLA's, here
numpy's 1/sqrt), and cos/sin are the platform's fp32 functions; a 1-ulp fp32
difference can move a bf16 rounding by one bf16 ulp. Everything else is exact.
"""
from __future__ import annotations

import numpy as np

from .attention_oracle import bf16_round


def rms_norm(x: np.ndarray, scale: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """bf16-valued float32 result of RMSNorm over the last axis."""
    x32 = np.asarray(x, dtype=np.float32)
    var = np.mean(np.square(x32), axis=-1, keepdims=True, dtype=np.float32)
    normed = x32 * (np.float32(1.0) / np.sqrt(var + np.float32(eps)))
    return bf16_round(bf16_round(normed) * bf16_round(np.asarray(scale, dtype=np.float32)))


def axis_freqs(seq_len: int, dim: int, theta: float = 10000.0):
    inv_freq = np.float32(1.0) / np.power(np.float32(theta), np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim))
    angles = np.outer(np.arange(seq_len, dtype=np.float32), inv_freq).astype(np.float32)
    return np.cos(angles), np.sin(angles)


def create_rope3d_freqs(t: int, h: int, w: int, head_dim: int, theta: float = 10000.0, max_seq_len: int = 1024):
    """(cos, sin), each (t*h*w, head_dim // 2) float32."""
    c = head_dim // 2
    dim_t, dim_h, dim_w = c - 2 * (c // 3), c // 3, c // 3
    ct, st = axis_freqs(max_seq_len, 2 * dim_t, theta)
    ch, sh = axis_freqs(max_seq_len, 2 * dim_h, theta)
    cw, sw = axis_freqs(max_seq_len, 2 * dim_w, theta)

    def grid(ft, fh, fw):
        gt = np.broadcast_to(ft[:t, None, None, :], (t, h, w, dim_t))
        gh = np.broadcast_to(fh[None, :h, None, :], (t, h, w, dim_h))
        gw = np.broadcast_to(fw[None, None, :w, :], (t, h, w, dim_w))
        return np.concatenate([gt, gh, gw], axis=-1).reshape(t * h * w, c)

    return grid(ct, ch, cw), grid(st, sh, sw)


def apply_rope3d(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x (B, S, H, D) -> bf16-valued float32, tables (S, D // 2)."""
    x32 = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)[None, :, None, :]
    s = np.asarray(sin, dtype=np.float32)[None, :, None, :]
    x1, x2 = x32[..., 0::2], x32[..., 1::2]
    out1 = x1 * c - x2 * s
    out2 = x2 * c + x1 * s
    out = np.stack([out1, out2], axis=-1).reshape(x32.shape)
    return bf16_round(out.astype(np.float32))


def qk_norm_rope(x: np.ndarray, scale, cos, sin, num_heads: int, eps: float = 1e-6) -> np.ndarray:
    """Wan's q/k prologue: RMSNorm over the whole row, reshape to heads, rope."""
    B, S, L = x.shape
    y = rms_norm(x, scale, eps) if scale is not None else np.asarray(x, dtype=np.float32)
    y = y.reshape(B, S, num_heads, L // num_heads)
    return apply_rope3d(y, cos, sin) if cos is not None else y


# ------------------------------------------------ neighbourhood-attention block
def default_rope_dim_split(head_dim: int):
    d_t = (head_dim // 4) // 2 * 2
    d_hw = (head_dim - d_t) // 2
    if d_hw % 2 != 0:
        d_t -= 2
        d_hw = (head_dim - d_t) // 2
    return d_t, d_hw, d_hw


def rope_inv_freqs(dim: int, base: float = 10000.0) -> np.ndarray:
    exponents = np.arange(0, dim, 2, dtype=np.float64) / dim
    return (1.0 / np.power(float(base), exponents)).astype(np.float32)


def apply_abs_rope_axis(xc: np.ndarray, pos: np.ndarray, inv: np.ndarray, axis: int) -> np.ndarray:
    """fp32 rotation of the (even, odd) pairs of the chunk xc (..., d) by
    pos (along `axis`) times inv."""
    xe, xo = xc[..., 0::2], xc[..., 1::2]
    shape = [1] * xc.ndim
    shape[axis] = pos.shape[0]
    shape[-1] = inv.shape[0]
    ang = (pos[:, None].astype(np.float32) * inv[None, :]).astype(np.float32).reshape(shape)
    c, s = np.cos(ang), np.sin(ang)
    out = np.empty_like(xc)
    out[..., 0::2] = xe * c - xo * s
    out[..., 1::2] = xe * s + xo * c
    return out


def apply_abs_rope3d(x: np.ndarray, rope_split=None, base: float = 10000.0) -> np.ndarray:
    """x (B, T, H, W, NH, HD) -> bf16-valued float32, rotated at arange
    positions on each axis."""
    x32 = np.asarray(x, dtype=np.float32)
    _, T, H, W, _, HD = x32.shape
    d_t, d_h, d_w = rope_split or default_rope_dim_split(HD)
    out = np.concatenate([
        apply_abs_rope_axis(x32[..., :d_t], np.arange(T), rope_inv_freqs(d_t, base), 1),
        apply_abs_rope_axis(x32[..., d_t:d_t + d_h], np.arange(H), rope_inv_freqs(d_h, base), 2),
        apply_abs_rope_axis(x32[..., d_t + d_h:], np.arange(W), rope_inv_freqs(d_w, base), 3),
    ], axis=-1)
    return bf16_round(out.astype(np.float32))


def create_abs_rope3d_freqs(t: int, h: int, w: int, head_dim: int, rope_split=None, base: float = 10000.0):
    """Per-token (cos, sin) tables, each (t*h*w, head_dim // 2) float32, of
    the same rotation (the layout the GPU kernel reads)."""
    d_t, d_h, d_w = rope_split or default_rope_dim_split(head_dim)

    def ang(n, d):
        return (np.arange(n, dtype=np.float32)[:, None] * rope_inv_freqs(d, base)[None, :]).astype(np.float32)

    at, ah, aw = ang(t, d_t), ang(h, d_h), ang(w, d_w)
    a = np.concatenate([
        np.broadcast_to(at[:, None, None, :], (t, h, w, d_t // 2)),
        np.broadcast_to(ah[None, :, None, :], (t, h, w, d_h // 2)),
        np.broadcast_to(aw[None, None, :, :], (t, h, w, d_w // 2)),
    ], axis=-1).reshape(t * h * w, head_dim // 2)
    return np.cos(a), np.sin(a)


def na3d_qk_norm_rope(x: np.ndarray, scale, post_scale: float = 1.0, rope: bool = True, eps: float = 1e-6,
                      rope_split=None, base: float = 10000.0) -> np.ndarray:
    """Per-head RMSNorm (skipped when scale is None) -> times bf16(post_scale)
    in bf16 -> absolute RoPE (skipped when rope is False), x (B,T,H,W,NH,HD)."""
    y = rms_norm(x, scale, eps) if scale is not None else np.asarray(x, dtype=np.float32)
    if post_scale != 1.0:
        y = bf16_round(y * bf16_round(np.float32(post_scale)))
    return apply_abs_rope3d(y, rope_split, base) if rope else y
