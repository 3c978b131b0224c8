"""CPU oracle for the DiT attention hot path (numpy restatement).

TEST INFRASTRUCTURE ONLY. Nothing in the product (`vidax_amd`) imports this
module; only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may use it, and only as the checker (or, for the baseline, as the
timed CPU restatement). The product path fails loudly when its HIP library is
missing instead of falling back to anything here.

What it restates (semantics, not code; the reference is JAX and cannot be
imported in this environment -- jax/jaxlib are absent):

* Full attention -- `src/vidax/core/attention.py:212-288` (flash path:
  softmax(sm_scale * q k^T [+ ab]) v over (B, S, H, D) tensors, padded keys
  excluded through segment ids at :272-278), :321-338 (`local_attention`,
  default scale 1/sqrt(D) at :335), :467-533 (`dot_product_attention`,
  default scale :524, additive `bias` broadcast to (B, H, Sq, Sk) at :280-283).
* Key-only masking -- `src/vidax/models/hunyuan_video/common/dit_layers.py`
  :150-190 (segment ids: every query row is segment 1, key j is segment
  key_valid[b, j]) and the dense restatement at :331-337 (fp32 logits *
  scale + (0 or -1e9) per key, fp32 softmax, weights cast to v's dtype).
  Cosmos3's (B, 1, 1, Sk) `-inf` key bias (`src/vidax/models/cosmos3/
  dit_layers.py:124-135`) is the same key-only mask in additive form.
* 3D neighbourhood attention -- `src/vidax/models/ltx2_5/diffusion_vae.py`
  :152-164 (`_window_start`: K' = min(K, L), start = clip(i - K'//2, 0,
  L - K')), :179-234 (`neighborhood_attention_3d`: per query, softmax over
  the kt'*kh'*kw' window keys of q.k with q pre-scaled by the caller at :265;
  logits einsum in the input dtype at :222, fp32 softmax, weights cast to
  v's dtype at :223).

A query row whose keys are all masked is defined here (and in the kernels)
to produce zeros; the reference never produces such a row at its call sites
and its output there is library-dependent (parity unpinned for that case).

bf16 is handled as float32 values that are exactly representable in bf16
(round-to-nearest-even), since numpy has no bfloat16 dtype.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_round",
    "bf16_to_bits",
    "bits_to_f32",
    "window_start",
    "window_indices",
    "attention",
    "attention_rows",
    "na3d",
    "na3d_loops",
    "make_flash_inputs",
    "make_na3d_inputs",
]


# ---------------------------------------------------------------- bf16 helpers
def bf16_to_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns, round to nearest even (NaN kept NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = 0x7FC0
    return out


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (RNE), returned as float32."""
    return bits_to_f32(bf16_to_bits(x))


# ---------------------------------------------------------- NATTEN windows
def window_start(length: int, kernel: int) -> np.ndarray:
    """Per-position window start along one axis.

    Follows `src/vidax/models/ltx2_5/diffusion_vae.py:152-164`: the kernel is
    clamped to the axis length first (K' = min(K, L)), then the window
    [start, start + K') is centred on i and shifted inwards at the borders,
    start = clip(i - K'//2, 0, L - K').
    """
    if length < 1 or kernel < 1:
        raise ValueError("length and kernel must be >= 1")
    k = min(kernel, length)
    i = np.arange(length)
    return np.clip(i - k // 2, 0, length - k)


def window_indices(length: int, kernel: int) -> np.ndarray:
    """(length, K') array of the key positions each query position attends."""
    k = min(kernel, length)
    return window_start(length, kernel)[:, None] + np.arange(k)[None, :]


# ------------------------------------------------------------ full attention
def _key_allowed(b: int, sk: int, kv_len, key_valid, key_bias):
    """Additive per-key term (0 / -inf / bias) for batch item b, float64."""
    add = np.zeros(sk, dtype=np.float64)
    if kv_len is not None:
        n = int(np.clip(kv_len[b], 0, sk))
        add[n:] = -np.inf
    if key_valid is not None:
        add[~np.asarray(key_valid[b, :sk]).astype(bool)] = -np.inf
    if key_bias is not None:
        add = add + np.asarray(key_bias[b, :sk], dtype=np.float64)
    return add


def _softmax_rows(logits: np.ndarray) -> np.ndarray:
    """Row softmax with fully masked rows mapped to zero weights."""
    m = np.max(logits, axis=-1, keepdims=True)
    dead = ~np.isfinite(m)
    m = np.where(dead, 0.0, m)
    e = np.exp(logits - m)
    s = np.sum(e, axis=-1, keepdims=True)
    w = e / np.where(s > 0, s, 1.0)
    return np.where(dead, 0.0, w)


def attention(q, k, v, scale=None, kv_len=None, key_valid=None, key_bias=None,
              acc=np.float64, weights_dtype_round=False, q_block=2048, bias=None):
    """softmax(scale * q k^T + key_mask) v for (B, Sq, H, D) / (B, Sk, H, D).

    Key masks are key-only: `kv_len` (B,) prefix lengths, `key_valid` (B, Sk)
    booleans, `key_bias` (B, Sk) additive logits (may hold -inf). Computed in
    `acc` precision; `weights_dtype_round=True` rounds the softmax weights to
    bf16 before the PV product, as the Hunyuan dense restatement does
    (`hunyuan_video/common/dit_layers.py:336`). `bias`, broadcastable to
    (B, H, Sq, Sk), is added to the scaled logits as the reference's
    non-kernel path does with a bias or a 0 / -inf boolean mask
    (`src/vidax/core/attention.py:533`, `wan/common/t5.py:40-68`).
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = D ** -0.5
    out = np.zeros((B, Sq, H, D), dtype=acc)
    full = None
    if bias is not None:
        full = np.broadcast_to(np.asarray(bias, dtype=np.float64), (B, H, Sq, Sk))
    for b in range(B):
        add = _key_allowed(b, Sk, kv_len, key_valid, key_bias).astype(acc)
        for h in range(H):
            kk = k[b, :, h, :].astype(acc)
            vv = v[b, :, h, :].astype(acc)
            for s0 in range(0, Sq, q_block):
                qq = q[b, s0:s0 + q_block, h, :].astype(acc)
                logits = (qq @ kk.T) * acc(scale) + add[None, :]
                if full is not None:
                    logits = logits + full[b, h, s0:s0 + q_block].astype(acc)
                w = _softmax_rows(logits)
                if weights_dtype_round:
                    w = bf16_round(w.astype(np.float32)).astype(acc)
                out[b, s0:s0 + q_block, h, :] = w @ vv
    return out


def attention_rows(q, k, v, rows, scale=None, kv_len=None, key_valid=None, key_bias=None,
                   acc=np.float64):
    """Oracle output for a subset of query rows only: (B, len(rows), H, D).

    Each output row depends only on its own query row and all keys, so this
    is exact for the chosen rows and lets full-size configurations be checked
    without the full O(Sq * Sk) work.
    """
    rows = np.asarray(rows)
    return attention(np.asarray(q)[:, rows], k, v, scale=scale, kv_len=kv_len,
                     key_valid=key_valid, key_bias=key_bias, acc=acc)


# ------------------------------------------------- neighbourhood attention
def na3d(q, k, v, kernel_size, scale=1.0, acc=np.float64, round_logits_bf16=False,
         round_weights_bf16=False, ty_rows=None):
    """3D neighbourhood attention over (B, T, H, W, NH, D) tensors.

    Window gather per axis (`window_indices`), then per query a softmax over
    its kt'*kh'*kw' keys. `scale` multiplies the logits (the reference's
    caller pre-scales q and passes no scale, i.e. 1.0). The optional rounding
    flags reproduce the reference's dtype points (bf16 logits, bf16 weights;
    `diffusion_vae.py:222-223`). `ty_rows`, a list of (t, y) query rows,
    restricts the computation to those rows (others are left at zero); each
    output row depends only on its own queries, so the subset is exact.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    B, T, Hs, W, NH, D = q.shape
    kt, kh, kw = kernel_size
    it = window_indices(T, kt)   # (T, kt')
    ih = window_indices(Hs, kh)  # (Hs, kh')
    iw = window_indices(W, kw)   # (W, kw')
    out = np.zeros(q.shape, dtype=acc)
    rows = [(t, y) for t in range(T) for y in range(Hs)] if ty_rows is None else list(ty_rows)
    for b in range(B):
        for t, y in rows:
            qq = q[b, t, y].astype(acc)                      # (W, NH, D)
            # keys: (kt', kh', W, kw', NH, D)
            kk = k[b][np.ix_(it[t], ih[y])]                   # (kt', kh', W, NH, D)
            vv = v[b][np.ix_(it[t], ih[y])]
            kk = kk[:, :, iw]                                 # (kt', kh', W, kw', NH, D)
            vv = vv[:, :, iw]
            kk = np.moveaxis(kk, 2, 0).reshape(W, -1, NH, D).astype(acc)
            vv = np.moveaxis(vv, 2, 0).reshape(W, -1, NH, D).astype(acc)
            logits = np.einsum("wnd,wknd->wnk", qq, kk) * acc(scale)
            if round_logits_bf16:
                logits = bf16_round(logits.astype(np.float32)).astype(acc)
            w = _softmax_rows(logits)
            if round_weights_bf16:
                w = bf16_round(w.astype(np.float32)).astype(acc)
            out[b, t, y] = np.einsum("wnk,wknd->wnd", w, vv)
    return out


def na3d_loops(q, k, v, kernel_size, scale=1.0):
    """Pure-Python brute force of the same definition, for tiny grids only.

    For every query position and head, enumerate the window explicitly with
    the clamp formula and evaluate the softmax in float64.
    """
    B, T, Hs, W, NH, D = q.shape
    kt, kh, kw = (min(kernel_size[0], T), min(kernel_size[1], Hs), min(kernel_size[2], W))
    out = np.zeros(q.shape, dtype=np.float64)

    def start(i, L, K):
        return min(max(i - K // 2, 0), L - K)

    for b in range(B):
        for t in range(T):
            for y in range(Hs):
                for x in range(W):
                    keys = [(tt, yy, xx)
                            for tt in range(start(t, T, kt), start(t, T, kt) + kt)
                            for yy in range(start(y, Hs, kh), start(y, Hs, kh) + kh)
                            for xx in range(start(x, W, kw), start(x, W, kw) + kw)]
                    for n in range(NH):
                        qv = q[b, t, y, x, n].astype(np.float64)
                        lg = np.array([scale * float(qv @ k[b, tt, yy, xx, n].astype(np.float64))
                                       for (tt, yy, xx) in keys])
                        w = np.exp(lg - lg.max())
                        w /= w.sum()
                        acc = np.zeros(D)
                        for wi, (tt, yy, xx) in zip(w, keys):
                            acc += wi * v[b, tt, yy, xx, n].astype(np.float64)
                        out[b, t, y, x, n] = acc
    return out


# ------------------------------------------------------------ inputs
def na3d_dense(q, k, v, kernel_size, scale=1.0, acc=np.float64, ty_rows=None):
    """na3d restated for whole grids: the same windows, computed per (t, y)
    query row as two dense matrix products over the row's key box.

    For query row (t, y) every query's window lies in the box of key rows
    it[t] x ih[y] (all W x positions); each query (x) keeps the kw' x
    positions iw[x] of every box row, so masking the rest to -inf before the
    softmax gives exactly its kt'*kh'*kw' keys (`diffusion_vae.py:152-234`).
    The products run on BLAS, over blocks of 16 queries along x (window
    starts grow with x, so a block's windows span x positions [start(x0),
    start(x1 - 1) + kw')), which makes the whole 21x45x80x24 grid a matter
    of seconds. `ty_rows` as in na3d (other rows left at zero).
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    B, T, Hs, W, NH, D = q.shape
    kt, kh, kw = kernel_size
    it = window_indices(T, kt)
    ih = window_indices(Hs, kh)
    iw = window_indices(W, kw)
    kw_ = iw.shape[1]
    nbox = it.shape[1] * ih.shape[1]
    XB = 16
    out = np.zeros(q.shape, dtype=acc)
    rows = [(t, y) for t in range(T) for y in range(Hs)] if ty_rows is None else list(ty_rows)
    for b in range(B):
        kb = np.ascontiguousarray(np.moveaxis(k[b], 3, 0), dtype=acc)        # (NH, T, Hs, W, D)
        vb = np.ascontiguousarray(np.moveaxis(v[b], 3, 0), dtype=acc)
        for t, y in rows:
            qq = np.ascontiguousarray(np.moveaxis(q[b, t, y], 1, 0), dtype=acc)   # (NH, W, D)
            tt, yy = it[t][:, None], ih[y][None, :]
            kbox = kb[:, tt, yy]                                                # (NH, kt', kh', W, D)
            vbox = vb[:, tt, yy]
            for x0 in range(0, W, XB):
                x1 = min(W, x0 + XB)
                lo, hi = int(iw[x0, 0]), int(iw[x1 - 1, 0]) + kw_
                kk = kbox[:, :, :, lo:hi].reshape(NH, nbox * (hi - lo), D)
                vv = vbox[:, :, :, lo:hi].reshape(NH, nbox * (hi - lo), D)
                # allowed[x, j]: box column j (x position lo + j % (hi - lo)) is in query x's window
                xin = np.zeros((x1 - x0, hi - lo), dtype=bool)
                xin[np.arange(x1 - x0)[:, None], iw[x0:x1] - lo] = True
                allowed = np.tile(xin, (1, nbox))
                logits = np.matmul(qq[:, x0:x1], np.swapaxes(kk, 1, 2)) * acc(scale)   # (NH, xb, box keys)
                w = _softmax_rows(np.where(allowed[None], logits, -np.inf))
                out[b, t, y, x0:x1] = np.moveaxis(np.matmul(w, vv), 0, 1)              # (xb, NH, D)
    return out


def _normal_bf16(rng, shape):
    return bf16_round(rng.standard_normal(shape, dtype=np.float32))


def make_flash_inputs(B, Sq, Sk, H, D, seed, mask=None):
    """Seeded bf16-valued inputs (float32 arrays), draw order Q, K, V, mask.

    mask: None, ("kv_len", lo, hi) -> int32 (B,) uniform in [lo, hi], or
    ("tail_pad", lo, hi) -> key_valid (B, Sk) with the last p ~ U{lo..hi} keys
    invalid.
    """
    rng = np.random.default_rng(seed)
    q = _normal_bf16(rng, (B, Sq, H, D))
    k = _normal_bf16(rng, (B, Sk, H, D))
    v = _normal_bf16(rng, (B, Sk, H, D))
    extra = {}
    if mask is not None:
        kind, lo, hi = mask
        n = rng.integers(lo, hi + 1, size=B)
        if kind == "kv_len":
            extra["kv_len"] = n.astype(np.int32)
        elif kind == "tail_pad":
            kv = np.ones((B, Sk), dtype=bool)
            for b in range(B):
                if n[b] > 0:
                    kv[b, Sk - n[b]:] = False
            extra["key_valid"] = kv
        else:
            raise ValueError(kind)
    return q, k, v, extra


def make_na3d_inputs(B, T, Hs, W, NH, D, seed, prescale=True):
    """Seeded bf16-valued NA inputs; q is pre-scaled by D**-0.5 in float32 and
    rounded to bf16 again, as the reference's caller does (`diffusion_vae.py:265`)."""
    rng = np.random.default_rng(seed)
    q = _normal_bf16(rng, (B, T, Hs, W, NH, D))
    k = _normal_bf16(rng, (B, T, Hs, W, NH, D))
    v = _normal_bf16(rng, (B, T, Hs, W, NH, D))
    if prescale:
        q = bf16_round(q * np.float32(D ** -0.5))
    return q, k, v
