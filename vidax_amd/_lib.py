"""ctypes binding of libvx_attn.so (the C ABI in include/vx_attn.h).

torch is imported before the library is opened so that the library binds to
the HIP runtime torch already loaded (both resolve `libamdhip64.so.7`): device
pointers and the hipStream_t taken from torch are then valid in the kernels.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the dlopen below)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libvx_attn.so")

VX_OK = 0
VX_ERR_INVALID_ARGUMENT = 1
VX_ERR_UNSUPPORTED = 2
VX_ERR_LAUNCH = 3

EXPORTED_SYMBOLS = (
    "vx_abi_version",
    "vx_last_error",
    "vx_flash_attn_fwd",
    "vx_flash_attn_check",
    "vx_na3d_fwd",
    "vx_na3d_check",
    "vx_debug_inject_error",
    "vx_rmsnorm_rope_fwd",
    "vx_rmsnorm_rope_check",
    "vx_flash_attn_bias_fwd",
    "vx_flash_attn_bias_check",
    "vx_rmsnorm_scale_rope_fwd",
    "vx_rmsnorm_scale_rope_check",
    "vx_flash_attn_plan",
    "vx_na3d_plan",
    "vx_last_launch",
    "vx_na3d_qprep_fwd",
    "vx_na3d_qprep_check",
    "vx_na3d_qprep_axes_fwd",
    "vx_na3d_qprep_axes_check",
    "vx_flash_attn_ws_fwd",
    "vx_flash_attn_workspace_size",
    "vx_flash_attn_split_plan",
    "vx_flash_attn_noalloc_fwd",
    "vx_debug_clock_stamp",
)

_lock = threading.Lock()
_lib = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)

_FLASH_ARGS = [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32,
               _i64p, _i64p, _i64p, _i64p, _f32]
_NA3D_ARGS = [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32]
_FLASH_BIAS_ARGS = [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64p, _i32, _i32, _i32, _i32, _i32,
                    _i64p, _i64p, _i64p, _i64p, _f32]
_NA3D_QPREP_ARGS = [_p, _p, _p, _p] + [_i32] * 9 + [_p, _f32, _f32, _p, _p, _i64]
_NA3D_QPREP_AXES_ARGS = [_p, _p, _p, _p] + [_i32] * 9 + [_p, _f32, _f32, _p, _p, _i64, _i32p]
_PROLOGUE_ARGS = [_p, _p, _p, _f32, _i32, _p, _p, _i64, _i32, _i32, _i32, _i32, _i64p, _i64p]
_SCALED_PROLOGUE_ARGS = _PROLOGUE_ARGS[:5] + [_f32] + _PROLOGUE_ARGS[5:]


class VxError(RuntimeError):
    """A failure reported by the C ABI (code and message from vx_last_error)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"vx error {code}: {message}")
        self.code = code
        self.message = message


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"vidax_amd: {LIB_PATH} is missing; build it with "
                    "`python -m vidax_amd.build` (or __graft_entry__.build()). "
                    "There is no fallback implementation.")
            h = ctypes.CDLL(LIB_PATH)
            h.vx_abi_version.restype = _i32
            h.vx_abi_version.argtypes = []
            h.vx_last_error.restype = ctypes.c_char_p
            h.vx_last_error.argtypes = []
            h.vx_flash_attn_fwd.restype = _i32
            h.vx_flash_attn_fwd.argtypes = _FLASH_ARGS + [_p]
            h.vx_flash_attn_check.restype = _i32
            h.vx_flash_attn_check.argtypes = _FLASH_ARGS
            h.vx_na3d_fwd.restype = _i32
            h.vx_na3d_fwd.argtypes = _NA3D_ARGS + [_p]
            h.vx_na3d_check.restype = _i32
            h.vx_na3d_check.argtypes = _NA3D_ARGS
            h.vx_flash_attn_bias_fwd.restype = _i32
            h.vx_flash_attn_bias_fwd.argtypes = _FLASH_BIAS_ARGS + [_p]
            h.vx_flash_attn_bias_check.restype = _i32
            h.vx_flash_attn_bias_check.argtypes = _FLASH_BIAS_ARGS
            h.vx_rmsnorm_rope_fwd.restype = _i32
            h.vx_rmsnorm_rope_fwd.argtypes = _PROLOGUE_ARGS + [_p]
            h.vx_rmsnorm_rope_check.restype = _i32
            h.vx_rmsnorm_rope_check.argtypes = _PROLOGUE_ARGS
            h.vx_rmsnorm_scale_rope_fwd.restype = _i32
            h.vx_rmsnorm_scale_rope_fwd.argtypes = _SCALED_PROLOGUE_ARGS + [_p]
            h.vx_rmsnorm_scale_rope_check.restype = _i32
            h.vx_rmsnorm_scale_rope_check.argtypes = _SCALED_PROLOGUE_ARGS
            h.vx_debug_inject_error.restype = None
            h.vx_debug_inject_error.argtypes = [_i32]
            h.vx_flash_attn_plan.restype = _i32
            h.vx_flash_attn_plan.argtypes = [_i32] * 6 + [ctypes.c_char_p, _i32]
            h.vx_na3d_plan.restype = _i32
            h.vx_na3d_plan.argtypes = [_i32] * 7 + [ctypes.c_char_p, _i32]
            h.vx_na3d_qprep_fwd.restype = _i32
            h.vx_na3d_qprep_fwd.argtypes = _NA3D_QPREP_ARGS + [_p]
            h.vx_na3d_qprep_check.restype = _i32
            h.vx_na3d_qprep_check.argtypes = _NA3D_QPREP_ARGS
            h.vx_na3d_qprep_axes_fwd.restype = _i32
            h.vx_na3d_qprep_axes_fwd.argtypes = _NA3D_QPREP_AXES_ARGS + [_p]
            h.vx_na3d_qprep_axes_check.restype = _i32
            h.vx_na3d_qprep_axes_check.argtypes = _NA3D_QPREP_AXES_ARGS
            h.vx_flash_attn_ws_fwd.restype = _i32
            h.vx_flash_attn_ws_fwd.argtypes = _FLASH_ARGS + [_p, _i64, _p]
            h.vx_flash_attn_noalloc_fwd.restype = _i32
            h.vx_flash_attn_noalloc_fwd.argtypes = _FLASH_ARGS + [_p]
            h.vx_flash_attn_workspace_size.restype = _i64
            h.vx_flash_attn_workspace_size.argtypes = [_i32] * 5
            h.vx_flash_attn_split_plan.restype = _i32
            h.vx_flash_attn_split_plan.argtypes = [_i32] * 6 + [ctypes.POINTER(_i32), ctypes.POINTER(_i32),
                                                               ctypes.POINTER(_i64)]
            h.vx_debug_clock_stamp.restype = _i32
            h.vx_debug_clock_stamp.argtypes = [_p, _i32, ctypes.POINTER(_i32), _p]
            h.vx_last_launch.restype = ctypes.c_char_p
            h.vx_last_launch.argtypes = []
            _lib = h
    return _lib


def last_error() -> str:
    return lib().vx_last_error().decode("utf-8", "replace")


def last_launch() -> str:
    """Kernel launched by the last successful vx_*_fwd call on this thread."""
    return lib().vx_last_launch().decode("utf-8", "replace")


def flash_plan(batch: int, seq_q: int, seq_k: int, num_heads: int, head_dim: int, mask_kind: int) -> str:
    """Kernel vx_flash_attn_fwd would launch for this shape (host-side plan)."""
    buf = ctypes.create_string_buffer(64)
    raise_for(lib().vx_flash_attn_plan(batch, seq_q, seq_k, num_heads, head_dim, mask_kind, buf, 64))
    return buf.value.decode()


_FAKE_PTR = 1 << 20  # a 16-byte aligned address for host-only checks (never dereferenced)


def flash_shape_check(batch: int, seq_q: int, seq_k: int, num_heads: int, head_dim: int):
    """(code, message) of vx_flash_attn_check for contiguous tensors of this
    shape, without a GPU: VX_OK, or VX_ERR_UNSUPPORTED for a shape the
    kernels do not take (e.g. a head dim other than 64 or 128)."""
    rc = lib().vx_flash_attn_check(_FAKE_PTR, _FAKE_PTR, _FAKE_PTR, _FAKE_PTR, None, None, None, 0,
                                   int(batch), int(seq_q), int(seq_k), int(num_heads), int(head_dim),
                                   None, None, None, None, ctypes.c_float(1.0))
    return rc, ("" if rc == VX_OK else last_error())


def na3d_plan(t: int, h: int, w: int, head_dim: int, kernel_t: int, kernel_h: int, kernel_w: int) -> str:
    """Kernel vx_na3d_fwd would launch for this grid and window (host-side plan)."""
    buf = ctypes.create_string_buffer(64)
    raise_for(lib().vx_na3d_plan(t, h, w, head_dim, kernel_t, kernel_h, kernel_w, buf, 64))
    return buf.value.decode()


def raise_for(code: int) -> None:
    """Maps a non-zero C ABI return code to a Python exception."""
    if code == VX_OK:
        return
    msg = last_error()
    if code == VX_ERR_INVALID_ARGUMENT:
        raise ValueError(f"vidax_amd: {msg}")
    if code == VX_ERR_UNSUPPORTED:
        raise NotImplementedError(f"vidax_amd: {msg}")
    raise VxError(code, msg)


def strides2(strides) -> ctypes.Array:
    return (ctypes.c_int64 * 2)(*[int(s) for s in strides])


def strides3(strides) -> ctypes.Array:
    arr = (ctypes.c_int64 * 3)(*[int(s) for s in strides])
    return arr
