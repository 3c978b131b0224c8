"""Attention entry points of vidax, re-exposed over the gfx950 HIP kernels.

Same names, arguments, layouts and masking semantics as the reference's
`src/vidax/core/attention.py` and `src/vidax/models/hunyuan_video/common/
dit_layers.py`, with torch tensors on the GPU standing in for jnp arrays
(q/k/v are (B, S, H, D) bfloat16 cuda tensors). Every call launches the HIP
kernel through the C ABI on torch's current stream; there is no other
implementation behind these functions, so a missing library or an unsupported
request raises instead of silently running something else.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from . import _lib

__all__ = [
    "flash_attention",
    "flash_kernel_name",
    "flash_supported",
    "local_attention",
    "dot_product_attention",
    "masked_self_attention",
]


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.dim() != 4:
            raise ValueError(f"{name} must be (B, S, H, D); got shape {tuple(t.shape)}")
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16; got {t.dtype}")
        if not t.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must have a contiguous head dim")
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    if q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2] or q.shape[3] != k.shape[3]:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree on B, H or D")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k and v must be on the same device")


# The kernel copies k and v tiles with 32-bit offsets: their sequence stride
# must stay within 2^24 elements (a contiguous (B, S, H, D) tensor has H * D).
_MAX_KV_SEQ_STRIDE = 1 << 24


def _aligned(t: torch.Tensor, max_seq_stride: Optional[int] = None) -> torch.Tensor:
    """Tensor usable by the kernels: 16-byte aligned with strides in multiples
    of 8 (and, for k and v, a sequence stride within the kernel's limit);
    otherwise a contiguous copy."""
    ok = t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:3])
    if max_seq_stride is not None and t.stride(1) > max_seq_stride:
        ok = False
    return t if ok else t.contiguous()


def _mask_rows(x: torch.Tensor, sk: int, dtype: torch.dtype, fill) -> torch.Tensor:
    """(B, Sk) -> (B, round_up(Sk, 64)) contiguous copy in `dtype`, padded with `fill`
    (the kernel stages the mask in whole 64-key tiles)."""
    b = x.shape[0]
    width = (sk + 63) // 64 * 64
    out = torch.full((b, width), fill, dtype=dtype, device=x.device)
    out[:, :sk] = x.to(dtype)
    return out


def _last_valid_plus_one(valid: torch.Tensor) -> torch.Tensor:
    """(B, Sk) bool -> int32 (B,) index of the last valid key + 1 (0 if none), on device."""
    sk = valid.shape[-1]
    pos = torch.arange(1, sk + 1, device=valid.device, dtype=torch.int32)
    return (valid.to(torch.int32) * pos).amax(dim=-1).to(torch.int32).contiguous()


def _full_bias(bias, B: int, H: int, Sq: int, Sk: int, dev) -> Tuple[torch.Tensor, Tuple[int, int, int]]:
    """A bias broadcastable to (B, H, Sq, Sk) -- every dim 1 or full, as
    `jnp.broadcast_to` accepts (`src/vidax/core/attention.py:282,533`) -- as
    the kernel reads it: fp32, keys contiguous, every query row readable for
    round_up(Sk, 64) keys, 16-byte aligned, strides multiples of 4 (0 for
    broadcast dims). A key dim of 1 is expanded; copies only when the given
    tensor does not already have that form."""
    x = torch.as_tensor(bias, device=dev)
    while x.dim() < 4:
        x = x.unsqueeze(0)
    if x.dim() != 4 or any(x.shape[i] not in (1, n) for i, n in enumerate((B, H, Sq, Sk))):
        raise ValueError(f"bias of shape {tuple(bias.shape)} is not broadcastable to (B, H, Sq, Sk) = "
                         f"({B}, {H}, {Sq}, {Sk})")
    x = x.to(torch.float32)
    if x.shape[3] != Sk:
        x = x.expand(x.shape[0], x.shape[1], x.shape[2], Sk)
    width = (Sk + 63) // 64 * 64
    ok = (x.stride(3) == 1 and Sk == width and x.data_ptr() % 16 == 0 and
          all(x.stride(i) % 4 == 0 for i in range(3)))
    if not ok:
        pad = torch.zeros(x.shape[:3] + (width,), dtype=torch.float32, device=dev)
        pad[..., :Sk] = x
        x = pad
    strides = tuple(0 if x.shape[i] == 1 else x.stride(i) for i in range(3))
    return x, strides


def flash_supported(batch: int, seq_q: int, seq_k: int, num_heads: int, head_dim: int) -> bool:
    """Whether the flash kernels take q (batch, seq_q, num_heads, head_dim)
    against keys of seq_k: a host-only check (the C ABI's
    vx_flash_attn_check), so a caller can decide at trace time. The kernels
    take head dims 64 and 128; the reference's own dispatcher keeps
    `jax.nn.dot_product_attention` for shapes its kernel cannot take
    (`src/vidax/core/attention.py:519-533`), e.g. CLIP's D=80
    (`wan/wan2_1/clip_vision.py:36-46`) and the Wan VAE's single D=384 head
    (`wan/common/vae_layers.py:100-110`), and a drop-in branch does the same."""
    return _lib.flash_shape_check(batch, seq_q, seq_k, num_heads, head_dim)[0] == _lib.VX_OK


def _require_supported(B: int, Sq: int, Sk: int, H: int, D: int) -> None:
    rc, msg = _lib.flash_shape_check(B, Sq, Sk, H, D)
    if rc == _lib.VX_ERR_UNSUPPORTED:
        raise NotImplementedError(
            f"vidax_amd: {msg}. This shape is outside the gfx950 flash kernels; the reference keeps "
            "jax.nn.dot_product_attention for it (src/vidax/core/attention.py:533), and a drop-in "
            "integration branches on vidax_amd.flash_supported(...) before calling these entry points")
    _lib.raise_for(rc)


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                    scale: Optional[float] = None,
                    kv_len: Optional[torch.Tensor] = None,
                    key_valid: Optional[torch.Tensor] = None,
                    key_bias: Optional[torch.Tensor] = None,
                    bias: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Non-causal flash attention with optional key-only masks and an
    optional additive bias that may also depend on head and query.

    q (B, Sq, H, D), k/v (B, Sk, H, D), bf16 on the GPU; returns (B, Sq, H, D).
    scale defaults to 1/sqrt(D) (`src/vidax/core/attention.py:335,524`).
    kv_len (B,) int: keys >= kv_len[b] masked (prefix form). key_valid
    (B, Sk) bool/int: general key validity. key_bias (B, Sk) float: additive
    logits (-inf masks). All masks broadcast over heads and query rows, as
    the reference's segment ids do (`hunyuan_video/common/dit_layers.py:183-186`).
    bias: fp32-convertible, broadcastable to (B, H, Sq, Sk), added to the
    scaled logits (T5's relative-position bias, `wan/common/t5.py:40-68`;
    0 / -inf from a boolean mask). It is read per query row from memory, so
    it suits the short sequences that use it.
    """
    _check_qkv(q, k, v)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    _require_supported(B, Sq, Sk, H, D)
    if scale is None:
        scale = D ** -0.5
    scale = float(scale)
    q = _aligned(q)
    k, v = _aligned(k, _MAX_KV_SEQ_STRIDE), _aligned(v, _MAX_KV_SEQ_STRIDE)
    if out is None:
        out = torch.empty((B, Sq, H, D), dtype=q.dtype, device=q.device)
    elif out.shape != (B, Sq, H, D) or out.dtype != q.dtype or out.stride(-1) != 1 or out.device != q.device:
        raise ValueError("out must be a (B, Sq, H, D) bf16 tensor with a contiguous head dim, on q's device")
    dev = q.device
    kv_len_t = key_valid_t = key_bias_t = None
    stride = 0
    if kv_len is not None:
        kv_len_t = torch.as_tensor(kv_len, device=dev).to(torch.int32).reshape(B).contiguous()
    if key_valid is not None:
        kvd = torch.as_tensor(key_valid, device=dev).reshape(B, Sk).to(torch.bool)
        key_valid_t = _mask_rows(kvd, Sk, torch.uint8, 0)
        stride = key_valid_t.shape[1]
    if key_bias is not None:
        kbd = torch.as_tensor(key_bias, device=dev).reshape(B, Sk).to(torch.float32)
        key_bias_t = _mask_rows(kbd, Sk, torch.float32, float("-inf"))
        stride = key_bias_t.shape[1]
    L = _lib.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    if bias is not None:
        fb, fbs = _full_bias(bias, B, H, Sq, Sk, dev)
        with torch.cuda.device(dev):
            rc = L.vx_flash_attn_bias_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                kv_len_t.data_ptr() if kv_len_t is not None else None,
                key_valid_t.data_ptr() if key_valid_t is not None else None,
                key_bias_t.data_ptr() if key_bias_t is not None else None,
                stride, fb.data_ptr(), _lib.strides3(fbs), B, Sq, Sk, H, D,
                _lib.strides3(q.stride()[:3]), _lib.strides3(k.stride()[:3]),
                _lib.strides3(v.stride()[:3]), _lib.strides3(out.stride()[:3]),
                ctypes.c_float(scale), ctypes.c_void_p(stream))
        _lib.raise_for(rc)
        return out
    with torch.cuda.device(dev):
        # grids whose last round would leave the device mostly idle split
        # that round's query tiles over two key halves (fp32 partials in a
        # workspace from torch's caching allocator)
        # (calls with a key bias never split: no workspace)
        ws_bytes = 0 if key_bias_t is not None else int(L.vx_flash_attn_workspace_size(B, Sq, Sk, H, D))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
        rc = L.vx_flash_attn_ws_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            kv_len_t.data_ptr() if kv_len_t is not None else None,
            key_valid_t.data_ptr() if key_valid_t is not None else None,
            key_bias_t.data_ptr() if key_bias_t is not None else None,
            stride, B, Sq, Sk, H, D,
            _lib.strides3(q.stride()[:3]), _lib.strides3(k.stride()[:3]),
            _lib.strides3(v.stride()[:3]), _lib.strides3(out.stride()[:3]),
            ctypes.c_float(scale), ws.data_ptr() if ws is not None else None, ws_bytes,
            ctypes.c_void_p(stream))
    _lib.raise_for(rc)
    return out


def flash_kernel_name(batch: int, seq_q: int, seq_k: int, num_heads: int, head_dim: int = 128,
                      mask_kind: int = 0, num_cus: Optional[int] = None) -> str:
    """Name of the kernel the library launches for this shape (the C ABI's
    launch plan: the gfx950 tile table or VIDAX_FLASH_BLOCK_SIZES). mask_kind:
    1 key validity, 2 key bias, 4 full bias (bits).

    Without num_cus: the kernel of vx_flash_attn_fwd, which never splits its
    keys. With num_cus (the device's compute units): the kernel of
    vx_flash_attn_ws_fwd given its workspace, as flash_attention calls it,
    i.e. flash_fwd_split_kernel<...> for the grids whose last round the key
    split evens out (vx_flash_attn_split_plan; never with a key or full bias)."""
    name = _lib.flash_plan(int(batch), int(seq_q), int(seq_k), int(num_heads), int(head_dim), int(mask_kind))
    if num_cus is not None and int(mask_kind) in (0, 1) and name.startswith("flash_fwd_kernel<"):
        items = ctypes.c_int32(0)
        key = ctypes.c_int32(0)
        nbytes = ctypes.c_int64(0)
        _lib.raise_for(_lib.lib().vx_flash_attn_split_plan(int(batch), int(seq_q), int(seq_k), int(num_heads),
                                                           int(head_dim), int(num_cus), ctypes.byref(items),
                                                           ctypes.byref(key), ctypes.byref(nbytes)))
        if items.value > 0:
            name = name.replace("flash_fwd_kernel<", "flash_fwd_split_kernel<")
    return name


def _single_device(mesh) -> None:
    """This build runs on one GPU: a mesh, if given, must hold one device."""
    if mesh is None:
        return
    size = getattr(mesh, "size", None)
    devices = getattr(mesh, "devices", None)
    if size is None and devices is not None:
        size = getattr(devices, "size", None)
    if size != 1:
        raise NotImplementedError(
            "vidax_amd runs attention on a single GPU; multi-device meshes "
            "(the reference's shard_map wrappers) are not part of this build")


def _key_only(x: torch.Tensor, B: int, Sk: int, what: str) -> Optional[torch.Tensor]:
    """Reduces a tensor broadcastable to (B, H, Sq, Sk) to (B, Sk) if it only
    varies along batch and key (a key dim of 1 broadcasts); returns None
    otherwise."""
    x = torch.as_tensor(x)
    while x.dim() < 4:
        x = x.unsqueeze(0)
    if x.dim() != 4 or x.shape[0] not in (1, B) or x.shape[3] not in (1, Sk):
        raise ValueError(f"{what} of shape {tuple(x.shape)} is not broadcastable to (B, H, Sq, Sk) with "
                         f"B={B}, Sk={Sk}")
    if x.shape[1] != 1 or x.shape[2] != 1:
        return None
    return x.expand(B, 1, 1, Sk).reshape(B, Sk)


def local_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    scale: Optional[float] = None) -> torch.Tensor:
    """Plain single-call attention (`src/vidax/core/attention.py:321-338`)."""
    head_dim = q.shape[-1]
    sm_scale = head_dim ** -0.5 if scale is None else scale
    return flash_attention(q, k, v, scale=sm_scale)


def dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          bias: Optional[torch.Tensor] = None,
                          mask: Optional[torch.Tensor] = None,
                          scale: Optional[float] = None,
                          mesh=None) -> torch.Tensor:
    """Full non-causal attention (`src/vidax/core/attention.py:467-533`).

    `bias` and `mask` are broadcastable to (B, H, Sq, Sk), as in the
    reference. Key-only forms -- shape (B or 1, 1, 1, Sk), e.g. Cosmos3's
    (B, 1, 1, Sk) -inf padding bias -- run in the flash kernel's key-mask
    path: the key loop is bounded by the last valid key, and the kernel
    classifies each 64-key tile itself (all-zero bias, all-valid tiles run
    unmasked), so no mask is inspected on the host. Head- or
    query-dependent ones -- T5's relative-position bias, causal masks, the
    reference's `jax.nn.dot_product_attention` fallback -- run in the same
    kernel with a per-(query, key) bias (a boolean mask becomes 0 / -inf).
    """
    _check_qkv(q, k, v)
    _single_device(mesh)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    _require_supported(B, Sq, Sk, H, D)
    sm_scale = D ** -0.5 if scale is None else scale
    key_bias = key_valid = kv_len = full = None
    valid = None
    if bias is not None:
        kb = _key_only(torch.as_tensor(bias, device=q.device), B, Sk, "bias")
        if kb is None:
            full = torch.as_tensor(bias, device=q.device).to(torch.float32)
        else:
            key_bias = kb.to(torch.float32)
            valid = key_bias > float("-inf")
    if mask is not None:
        km = _key_only(torch.as_tensor(mask, device=q.device), B, Sk, "mask")
        if km is None:
            m = torch.as_tensor(mask, device=q.device).to(torch.bool)
            add = torch.zeros(m.shape, dtype=torch.float32, device=q.device).masked_fill_(~m, float("-inf"))
            full = add if full is None else full + add
        else:
            key_valid = km.to(torch.bool)
            valid = key_valid if valid is None else (valid & key_valid)
    if valid is not None:
        kv_len = _last_valid_plus_one(valid)
    return flash_attention(q, k, v, scale=sm_scale, kv_len=kv_len, key_valid=key_valid,
                           key_bias=key_bias, bias=full)


def masked_self_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          key_valid: Optional[torch.Tensor] = None,
                          mesh=None, tp_sharded: bool = True) -> torch.Tensor:
    """Self-attention with an optional key-only validity mask, returning
    (B, S, H*D) (`src/vidax/models/hunyuan_video/common/dit_layers.py:264-337`).

    key_valid (B, S) bool/int marks valid keys; every query row (valid or
    not) attends exactly the valid keys, as the reference's segment ids do
    (q ids all 1, kv ids = key_valid; `dit_layers.py:183-186`). The reference
    documents valid keys as a prefix; any pattern is handled exactly here:
    the key loop stops at the last valid key, and tiles whose keys are all
    valid run the unmasked path (classified by the kernel, with no host
    synchronisation).
    """
    del tp_sharded  # selects a shard_map wrapper in the reference; one GPU here
    _check_qkv(q, k, v)
    _single_device(mesh)
    b, s, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    if key_valid is None:
        out = flash_attention(q, k, v, scale=scale)
    else:
        kv = torch.as_tensor(key_valid, device=q.device).reshape(b, k.shape[1]).to(torch.bool)
        kv_len = _last_valid_plus_one(kv)
        out = flash_attention(q, k, v, scale=scale, kv_len=kv_len, key_valid=kv)
    return out.reshape(b, s, h * d)
