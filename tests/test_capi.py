"""CPU tests of the C ABI: the library loads without a GPU, exports every
symbol include/vx_attn.h declares, and its argument checks, error codes,
messages and failure injection behave as documented. No kernel is launched:
every call here is rejected (or short-circuited by the injection hook) on the
host before any HIP call."""
import ctypes
import os
import re

import pytest

from vidax_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vx_attn.h")

A = 1 << 20  # a 16-byte aligned fake device address (never dereferenced)


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vx_\w+)\s*\(", text)))


def test_header_symbols_are_exported():
    L = _lib.lib()
    names = _declared()
    assert set(names) == set(_lib.EXPORTED_SYMBOLS)
    for n in names:
        assert hasattr(L, n), n


def test_abi_version():
    assert _lib.lib().vx_abi_version() == 10800


def _flash_check(**kw):
    args = dict(q=A, k=A, v=A, out=A, kv_len=None, key_valid=None, key_bias=None, stride=0,
                B=1, Sq=100, Sk=200, H=4, D=128, qs=None, ks=None, vs=None, os_=None, scale=0.088)
    args.update(kw)
    s3 = lambda s: None if s is None else _lib.strides3(s)
    return _lib.lib().vx_flash_attn_check(
        args["q"], args["k"], args["v"], args["out"], args["kv_len"], args["key_valid"],
        args["key_bias"], args["stride"], args["B"], args["Sq"], args["Sk"], args["H"], args["D"],
        s3(args["qs"]), s3(args["ks"]), s3(args["vs"]), s3(args["os_"]), ctypes.c_float(args["scale"]))


def test_flash_check_accepts_valid_arguments():
    assert _flash_check() == _lib.VX_OK
    assert _lib.last_error() == ""
    assert _flash_check(qs=(200 * 4 * 128, 4 * 128, 128)) == _lib.VX_OK
    assert _flash_check(key_valid=A, stride=256) == _lib.VX_OK
    assert _flash_check(key_bias=A, kv_len=A, stride=260) == _lib.VX_OK


@pytest.mark.parametrize("kw,code,frag", [
    (dict(q=None), _lib.VX_ERR_INVALID_ARGUMENT, "non-NULL"),
    (dict(out=A + 8), _lib.VX_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(B=0), _lib.VX_ERR_INVALID_ARGUMENT, ">= 1"),
    (dict(Sk=0), _lib.VX_ERR_INVALID_ARGUMENT, ">= 1"),
    (dict(H=70000), _lib.VX_ERR_INVALID_ARGUMENT, "65535"),
    (dict(D=96), _lib.VX_ERR_UNSUPPORTED, "head_dim"),
    (dict(scale=0.0), _lib.VX_ERR_INVALID_ARGUMENT, "scale"),
    (dict(scale=float("inf")), _lib.VX_ERR_INVALID_ARGUMENT, "scale"),
    (dict(scale=-1.0), _lib.VX_ERR_INVALID_ARGUMENT, "scale"),
    (dict(qs=(0, 4 * 128, 129)), _lib.VX_ERR_INVALID_ARGUMENT, "multiple of 8"),
    (dict(ks=(0, -512, 128)), _lib.VX_ERR_INVALID_ARGUMENT, "negative"),
    (dict(ks=(0, (1 << 24) + 8, 128)), _lib.VX_ERR_UNSUPPORTED, "2^24"),
    (dict(vs=(0, 1 << 25, 128)), _lib.VX_ERR_UNSUPPORTED, "2^24"),
    (dict(key_valid=A, stride=200), _lib.VX_ERR_INVALID_ARGUMENT, "key_mask_stride"),
    (dict(key_valid=A, stride=258), _lib.VX_ERR_INVALID_ARGUMENT, "key_mask_stride"),
    (dict(key_valid=A + 2, stride=256), _lib.VX_ERR_INVALID_ARGUMENT, "4-byte"),
    (dict(key_bias=A + 4, stride=256), _lib.VX_ERR_INVALID_ARGUMENT, "16-byte"),
    # a key bias enters the accumulator as bias / scale: 1 / scale must be finite
    (dict(key_bias=A, stride=256, scale=1e-39), _lib.VX_ERR_INVALID_ARGUMENT, "too small"),
])
def test_flash_check_rejects(kw, code, frag):
    assert _flash_check(**kw) == code
    assert frag in _lib.last_error()


def _na_check(**kw):
    args = dict(q=A, k=A, v=A, out=A, B=1, T=4, H=6, W=9, NH=2, D=128, kt=3, kh=5, kw=5, scale=1.0)
    args.update(kw)
    return _lib.lib().vx_na3d_check(args["q"], args["k"], args["v"], args["out"], args["B"], args["T"],
                                    args["H"], args["W"], args["NH"], args["D"], args["kt"], args["kh"],
                                    args["kw"], ctypes.c_float(args["scale"]))


def test_na3d_check():
    assert _na_check() == _lib.VX_OK
    assert _na_check(kt=100, kh=100, kw=100) == _lib.VX_OK          # clamped to the grid
    assert _na_check(W=200, kw=57) == _lib.VX_OK
    assert _na_check(W=200, kw=58) == _lib.VX_OK                     # any window (per-wave kernel)
    assert _na_check(W=300, kh=40, kw=199) == _lib.VX_OK
    assert _na_check(kt=0) == _lib.VX_ERR_INVALID_ARGUMENT
    assert _na_check(D=64) == _lib.VX_OK                             # LTX-2.5 VAE head dim
    assert _na_check(D=64, W=200, kw=25) == _lib.VX_OK
    assert _na_check(D=64, W=200, kw=27) == _lib.VX_OK
    assert _na_check(D=64, W=200, kw=99) == _lib.VX_OK
    assert _na_check(D=96) == _lib.VX_ERR_UNSUPPORTED
    assert _na_check(T=0) == _lib.VX_ERR_INVALID_ARGUMENT
    assert _na_check(k=A + 1) == _lib.VX_ERR_INVALID_ARGUMENT
    # one row of tokens (w * num_heads * head_dim elements) must stay below 2^30
    assert _na_check(W=8192, NH=1023, D=128, kw=5) == _lib.VX_OK
    assert _na_check(W=8192, NH=1024, D=128, kw=5) == _lib.VX_ERR_UNSUPPORTED
    assert _na_check(scale=float("nan")) == _lib.VX_ERR_INVALID_ARGUMENT


def test_fwd_rejects_before_launch():
    """Invalid arguments fail in the checker: no HIP call, so this runs without a GPU."""
    L = _lib.lib()
    rc = L.vx_flash_attn_fwd(A, A, A, A, None, None, None, 0, 1, 10, 10, 1, 96, None, None, None, None,
                             ctypes.c_float(1.0), None)
    assert rc == _lib.VX_ERR_UNSUPPORTED and "head_dim" in _lib.last_error()
    rc = L.vx_na3d_fwd(A, A, A, A, 1, 0, 1, 1, 1, 128, 1, 1, 1, ctypes.c_float(1.0), None)
    assert rc == _lib.VX_ERR_INVALID_ARGUMENT


def test_error_injection_short_circuits_launch():
    """The failure-injection hook returns its code after the argument checks
    and before any launch, so the error path can be exercised on a CPU host."""
    L = _lib.lib()
    L.vx_debug_inject_error(_lib.VX_ERR_LAUNCH)
    try:
        rc = L.vx_flash_attn_fwd(A, A, A, A, None, None, None, 0, 1, 10, 10, 1, 128, None, None, None, None,
                                 ctypes.c_float(1.0), None)
        assert rc == _lib.VX_ERR_LAUNCH and "injected" in _lib.last_error()
        with pytest.raises(_lib.VxError):
            _lib.raise_for(rc)
        rc = L.vx_na3d_fwd(A, A, A, A, 1, 2, 2, 2, 1, 128, 1, 1, 1, ctypes.c_float(1.0), None)
        assert rc == _lib.VX_ERR_LAUNCH
    finally:
        L.vx_debug_inject_error(0)
    # invalid arguments still win over the injection
    L.vx_debug_inject_error(_lib.VX_ERR_LAUNCH)
    try:
        rc = L.vx_flash_attn_fwd(None, A, A, A, None, None, None, 0, 1, 10, 10, 1, 128, None, None, None, None,
                                 ctypes.c_float(1.0), None)
        assert rc == _lib.VX_ERR_INVALID_ARGUMENT
    finally:
        L.vx_debug_inject_error(0)


def test_error_message_is_thread_local():
    import threading
    L = _lib.lib()
    assert _flash_check(D=96) == _lib.VX_ERR_UNSUPPORTED
    seen = {}

    def other():
        seen["msg"] = _lib.last_error()
    th = threading.Thread(target=other)
    th.start()
    th.join()
    assert seen["msg"] == ""
    assert "head_dim" in _lib.last_error()


def test_raise_for_maps_codes():
    _lib.raise_for(_lib.VX_OK)
    _flash_check(D=96)
    with pytest.raises(NotImplementedError):
        _lib.raise_for(_lib.VX_ERR_UNSUPPORTED)
    _flash_check(B=0)
    with pytest.raises(ValueError):
        _lib.raise_for(_lib.VX_ERR_INVALID_ARGUMENT)


def _prologue_check(**kw):
    args = dict(x=A, out=A + 4096, w=A, eps=1e-6, per_head=0, cos=A, sin=A, tab=64, B=1, S=10, H=4, D=128,
                xs=None, os_=None)
    args.update(kw)
    s2 = lambda s: None if s is None else _lib.strides2(s)
    return _lib.lib().vx_rmsnorm_rope_check(
        args["x"], args["out"], args["w"], ctypes.c_float(args["eps"]), args["per_head"], args["cos"],
        args["sin"], args["tab"], args["B"], args["S"], args["H"], args["D"], s2(args["xs"]), s2(args["os_"]))


def test_prologue_check_accepts_valid_arguments():
    assert _prologue_check() == _lib.VX_OK
    assert _prologue_check(w=None, per_head=1) == _lib.VX_OK
    assert _prologue_check(cos=None, sin=None, tab=0) == _lib.VX_OK
    assert _prologue_check(D=64, tab=32) == _lib.VX_OK
    assert _prologue_check(H=64) == _lib.VX_OK                              # rows of 8192
    assert _prologue_check(xs=(10 * 1536, 1536)) == _lib.VX_OK            # q slice of a fused qkv
    assert _prologue_check(out=A) == _lib.VX_OK                             # in place


@pytest.mark.parametrize("kw,code,frag", [
    (dict(x=None), _lib.VX_ERR_INVALID_ARGUMENT, "non-NULL"),
    (dict(out=A + 8), _lib.VX_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(S=0), _lib.VX_ERR_INVALID_ARGUMENT, ">= 1"),
    (dict(D=96), _lib.VX_ERR_UNSUPPORTED, "head_dim"),
    (dict(H=65), _lib.VX_ERR_UNSUPPORTED, "8192"),
    (dict(per_head=2), _lib.VX_ERR_INVALID_ARGUMENT, "per_head"),
    (dict(w=A + 4), _lib.VX_ERR_INVALID_ARGUMENT, "weight"),
    (dict(eps=-1.0), _lib.VX_ERR_INVALID_ARGUMENT, "eps"),
    (dict(sin=None), _lib.VX_ERR_INVALID_ARGUMENT, "both"),
    (dict(cos=A + 4), _lib.VX_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(tab=60), _lib.VX_ERR_INVALID_ARGUMENT, "rope_stride"),
    (dict(tab=66), _lib.VX_ERR_INVALID_ARGUMENT, "rope_stride"),
    (dict(xs=(5120, 12)), _lib.VX_ERR_INVALID_ARGUMENT, "multiples of 8"),
    (dict(out=A, os_=(8192, 1024)), _lib.VX_ERR_INVALID_ARGUMENT, "in-place"),
])
def test_prologue_check_rejects(kw, code, frag):
    assert _prologue_check(**kw) == code
    assert frag in _lib.last_error()


def _scaled_prologue_check(post_scale, **kw):
    args = dict(x=A, out=A + 4096, w=A, eps=1e-6, per_head=1, cos=A, sin=A, tab=32, B=1, S=10, H=4, D=64)
    args.update(kw)
    return _lib.lib().vx_rmsnorm_scale_rope_check(
        args["x"], args["out"], args["w"], ctypes.c_float(args["eps"]), args["per_head"], ctypes.c_float(post_scale),
        args["cos"], args["sin"], args["tab"], args["B"], args["S"], args["H"], args["D"], None, None)


def test_scaled_prologue_check():
    assert _scaled_prologue_check(0.125) == _lib.VX_OK
    assert _scaled_prologue_check(1.0) == _lib.VX_OK
    assert _scaled_prologue_check(-2.0, w=None) == _lib.VX_OK
    for bad in (float("inf"), float("nan")):
        assert _scaled_prologue_check(bad) == _lib.VX_ERR_INVALID_ARGUMENT
        assert "post_scale" in _lib.last_error()
    # the shared checks still apply
    assert _scaled_prologue_check(0.125, D=96) == _lib.VX_ERR_UNSUPPORTED


def _bias_check(bias=A, strides=(0, 256 * 256, 256), **kw):
    args = dict(q=A, k=A, v=A, out=A, kv_len=None, key_valid=None, key_bias=None, stride=0,
                B=1, Sq=100, Sk=200, H=4, D=128, scale=1.0)
    args.update(kw)
    return _lib.lib().vx_flash_attn_bias_check(
        args["q"], args["k"], args["v"], args["out"], args["kv_len"], args["key_valid"], args["key_bias"],
        args["stride"], bias, None if strides is None else _lib.strides3(strides), args["B"], args["Sq"],
        args["Sk"], args["H"], args["D"], None, None, None, None, ctypes.c_float(args["scale"]))


def test_flash_bias_check():
    assert _bias_check() == _lib.VX_OK
    assert _bias_check(strides=(0, 0, 0)) == _lib.VX_OK                  # fully broadcast
    assert _bias_check(bias=None) == _lib.VX_ERR_INVALID_ARGUMENT
    assert _bias_check(bias=A + 4) == _lib.VX_ERR_INVALID_ARGUMENT
    assert "aligned" in _lib.last_error()
    assert _bias_check(strides=(0, 256, 258)) == _lib.VX_ERR_INVALID_ARGUMENT
    assert "multiple of 4" in _lib.last_error()
    assert _bias_check(strides=None) == _lib.VX_ERR_INVALID_ARGUMENT
    assert _bias_check(D=64) == _lib.VX_OK
    assert _bias_check(D=96) == _lib.VX_ERR_UNSUPPORTED


def test_flash_kernel_name_follows_the_launch_rule():
    """The C ABI's launch plan (gfx950 tile table): 128-query workgroups for
    key sequences up to 1024 or fewer than 768 256-query tiles, else 256-query;
    short key sequences with no key masks but kv_len and at least 4096
    256-query tiles (at most 64 batch items) run the persistent kernel.
    (The GPU tests check that the launch itself matches the plan.)"""
    from vidax_amd.attention import flash_kernel_name
    assert flash_kernel_name(1, 32760, 32760, 40) == "flash_fwd_kernel<0, 128, 8>"
    assert flash_kernel_name(1, 119056, 119056, 24, 128, 1) == "flash_fwd_kernel<1, 128, 8>"
    assert flash_kernel_name(1, 7800, 7800, 12) == "flash_fwd_kernel<0, 128, 4>"      # 372 tiles
    assert flash_kernel_name(2, 32760, 512, 40) == "flash_stream_kernel<128>"        # short keys, 10240 tiles
    assert flash_kernel_name(2, 32760, 512, 40, 64) == "flash_stream_kernel<64>"
    assert flash_kernel_name(1, 65536, 1024, 16) == "flash_stream_kernel<128>"       # 4096 tiles
    assert flash_kernel_name(1, 65536, 1025, 16) == "flash_fwd_kernel<0, 128, 8>"    # keys above 1024
    assert flash_kernel_name(1, 65280, 1024, 16) == "flash_fwd_kernel<0, 128, 4>"    # 4080 tiles
    assert flash_kernel_name(65, 4096, 512, 4) == "flash_fwd_kernel<0, 128, 4>"      # 65 batch items
    assert flash_kernel_name(2, 32760, 512, 40, 128, 1) == "flash_fwd_kernel<1, 128, 4>"  # key validity
    assert flash_kernel_name(1, 200, 200, 4, 64, 4) == "flash_fwd_kernel<4, 64, 4>"
    # a per-(query, key) bias always runs 128-query workgroups
    assert flash_kernel_name(1, 32760, 32760, 40, 128, 5) == "flash_fwd_kernel<5, 128, 4>"
    # and so does key validity together with a key bias; each alone does not
    assert flash_kernel_name(1, 32760, 32760, 40, 128, 3) == "flash_fwd_kernel<3, 128, 4>"
    assert flash_kernel_name(1, 32760, 32760, 40, 128, 2) == "flash_fwd_kernel<2, 128, 8>"
    assert flash_kernel_name(3, 65536, 1025, 1) == "flash_fwd_kernel<0, 128, 8>"      # 768 tiles


def test_kv_views_with_oversized_sequence_stride_are_copied():
    """k/v views whose sequence stride exceeds the kernel's 2^24-element limit
    are handed over as contiguous copies; other aligned views pass as they are."""
    import torch
    from vidax_amd.attention import _MAX_KV_SEQ_STRIDE, _aligned
    big = _MAX_KV_SEQ_STRIDE + 8
    buf = torch.zeros(big + 16, dtype=torch.bfloat16)
    view = buf.as_strided((1, 2, 1, 8), (2 * big, big, 8, 1))
    assert _aligned(view) is view                          # q: no sequence-stride limit
    kv = _aligned(view, _MAX_KV_SEQ_STRIDE)
    assert kv is not view and kv.is_contiguous() and kv.stride(1) == 8
    small = torch.zeros((1, 4, 2, 64), dtype=torch.bfloat16)
    assert _aligned(small, _MAX_KV_SEQ_STRIDE) is small


def test_na3d_kernel_name_follows_the_launch_rule():
    """The C ABI's NA launch plan, by the clamped x window."""
    from vidax_amd.natten import na3d_kernel_name
    assert na3d_kernel_name(80, 7) == "na3d_pipe_kernel<16, 128>"
    assert na3d_kernel_name(80, 9, 64, height=4) == "na3d_pipe_kernel<16, 64>"   # 8x80 vs 4x96
    with pytest.raises(ValueError, match="height"):
        na3d_kernel_name(80, 9, 64)   # the height decides here
    # head dim 64, kw' <= 9: the tall bricks unless they pad the y-x plane more
    assert na3d_kernel_name(80, 7, 64, height=45) == "na3d_tall_kernel<64>"    # 48x80 vs 48x96
    assert na3d_kernel_name(80, 5, 64, height=44) == "na3d_tall_kernel<64>"    # 48x80 vs 44x96
    assert na3d_kernel_name(40, 7, 64, height=22) == "na3d_tall_kernel<64>"    # 24x48 vs 24x64
    assert na3d_kernel_name(20, 7, 64, height=11) == "na3d_pipe_kernel<16, 64>"  # 16x32 vs 12x32
    assert na3d_kernel_name(80, 7, 128, height=45) == "na3d_pipe_kernel<16, 128>"
    # head dim 128, kw' <= 9: two t planes per brick when the t window spans 2 or more
    assert na3d_kernel_name(80, 7, 128, height=45, depth=21, kernel_t=3) == "na3d_tstack_kernel<128>"
    assert na3d_kernel_name(80, 7, 128, depth=2, kernel_t=5) == "na3d_tstack_kernel<128>"    # kt' = 2
    assert na3d_kernel_name(80, 7, 128, depth=21, kernel_t=1) == "na3d_pipe_kernel<16, 128>"
    assert na3d_kernel_name(80, 7, 64, height=45, depth=21, kernel_t=3) == "na3d_tall_kernel<64>"
    assert na3d_kernel_name(80, 11, 64) == "na3d_tall_kernel<64>"        # 80 = 5 x 16, 96 in 32-wide bricks
    assert na3d_kernel_name(160, 11, 64) == "na3d_tall_wide_kernel<64>"  # 160 = 5 x 32
    assert na3d_kernel_name(104, 11, 64) == "na3d_tall_kernel<64>"       # 112 vs 128 columns
    assert na3d_kernel_name(24, 13, 64) == "na3d_tall_wide_kernel<64>"   # 32 columns either way
    # deep t windows (kt' >= 5) take the 32-wide bricks two t planes deep
    assert na3d_kernel_name(160, 11, 64, depth=33, kernel_t=11) == "na3d_deep_kernel<64>"
    assert na3d_kernel_name(160, 11, 64, depth=33, kernel_t=3) == "na3d_tall_wide_kernel<64>"
    assert na3d_kernel_name(160, 11, 64, depth=4, kernel_t=11) == "na3d_tall_wide_kernel<64>"  # kt' = 4
    assert na3d_kernel_name(80, 11, 64, depth=33, kernel_t=11) == "na3d_tall_kernel<64>"      # not 32-wide
    assert na3d_kernel_name(160, 11, 128, depth=33, kernel_t=11) == "na3d_tall_kernel<128>"
    assert na3d_kernel_name(160, 11) == "na3d_tall_kernel<128>"          # head dim 128: narrow bricks
    assert na3d_kernel_name(80, 13) == "na3d_tall_kernel<128>"
    assert na3d_kernel_name(12, 40) == "na3d_tall_kernel<128>"        # clamped to the grid width
    assert na3d_kernel_name(80, 14) == "na3d_pipe_kernel<32, 128>"
    assert na3d_kernel_name(80, 25, 64) == "na3d_pipe_kernel<32, 64>"
    assert na3d_kernel_name(80, 27) == "na3d_wave_kernel<128>"
    assert na3d_kernel_name(80, 27, 64) == "na3d_wave_kernel<64>"
    assert na3d_kernel_name(200, 99) == "na3d_wave_kernel<128>"


def test_small_scale_without_key_bias_is_accepted():
    assert _flash_check(scale=1e-39) == _lib.VX_OK


def _plan_in_subprocess(env_value, code):
    """Runs `code` in a fresh interpreter with VIDAX_FLASH_BLOCK_SIZES set
    (the library reads it once per process) and returns its stdout."""
    import subprocess
    import sys
    env = dict(os.environ)
    if env_value is None:
        env.pop("VIDAX_FLASH_BLOCK_SIZES", None)
    else:
        env["VIDAX_FLASH_BLOCK_SIZES"] = env_value
    res = subprocess.run([sys.executable, "-c", "import sys; sys.path.insert(0, %r)\n" % ROOT + code],
                         env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert res.returncode == 0, res.stdout
    return res.stdout.strip().splitlines()[-1]


_PLANS = ("from vidax_amd import _lib\n"
          "import ctypes\n"
          "b = ctypes.create_string_buffer(64)\n"
          "out = []\n"
          "for shape in [(1, 32760, 32760, 40), (2, 32760, 512, 40), (1, 7800, 7800, 12)]:\n"
          "    rc = _lib.lib().vx_flash_attn_plan(*shape, 128, 0, b, 64)\n"
          "    out.append(b.value.decode() if rc == 0 else 'rc=%d:%s' % (rc, _lib.last_error()))\n"
          "print('|'.join(out))\n")


@pytest.mark.parametrize("value,expect", [
    (None, ["flash_fwd_kernel<0, 128, 8>", "flash_stream_kernel<128>", "flash_fwd_kernel<0, 128, 4>"]),
    ("default", ["flash_fwd_kernel<0, 128, 8>", "flash_stream_kernel<128>", "flash_fwd_kernel<0, 128, 4>"]),
    (" DEFAULT ", ["flash_fwd_kernel<0, 128, 8>", "flash_stream_kernel<128>", "flash_fwd_kernel<0, 128, 4>"]),
    ("128,64,64", ["flash_fwd_kernel<0, 128, 4>"] * 3),
    ("256, 64, 64", ["flash_fwd_kernel<0, 128, 8>", "flash_stream_kernel<128>", "flash_fwd_kernel<0, 128, 8>"]),
])
def test_flash_block_sizes_override(value, expect):
    """VIDAX_FLASH_BLOCK_SIZES (the reference's override, core/attention.py:
    17-35) picks the query tile for every call; "default" keeps the table."""
    assert _plan_in_subprocess(value, _PLANS).split("|") == expect


@pytest.mark.parametrize("value,code,frag", [
    ("2048,1024,1024", _lib.VX_ERR_UNSUPPORTED, "key tiles of 64"),
    ("192,64,64", _lib.VX_ERR_UNSUPPORTED, "query tiles of 128 or 256"),
    ("256,64", _lib.VX_ERR_INVALID_ARGUMENT, "block_q,block_k_major,block_k"),
    ("256,64,64,1", _lib.VX_ERR_INVALID_ARGUMENT, "block_q,block_k_major,block_k"),
    ("big", _lib.VX_ERR_INVALID_ARGUMENT, "block_q,block_k_major,block_k"),
])
def test_flash_block_sizes_override_rejects(value, code, frag):
    """A malformed or unsupported override fails every flash plan and call
    (here through vx_flash_attn_check) with a message naming the variable."""
    code_str = ("from vidax_amd import _lib\n"
                "import ctypes\n"
                "b = ctypes.create_string_buffer(64)\n"
                "rc1 = _lib.lib().vx_flash_attn_plan(1, 100, 100, 2, 128, 0, b, 64)\n"
                "e1 = _lib.last_error()\n"
                "A = 1 << 20\n"
                "rc2 = _lib.lib().vx_flash_attn_check(A, A, A, A, None, None, None, 0, 1, 100, 100, 2, 128,"
                " None, None, None, None, ctypes.c_float(0.1))\n"
                "print('%d|%d|%s' % (rc1, rc2, e1))\n")
    rc1, rc2, msg = _plan_in_subprocess(value, code_str).split("|", 2)
    assert int(rc1) == code and int(rc2) == code
    assert frag in msg and "VIDAX_FLASH_BLOCK_SIZES" in msg


def test_last_launch_is_empty_before_any_launch():
    out = _plan_in_subprocess(None, "from vidax_amd import _lib\nprint(repr(_lib.last_launch()))\n")
    assert out == "''"


def test_full_bias_broadcasts_every_unit_dim():
    """Biases broadcast as jnp.broadcast_to does (core/attention.py:282,533):
    any dim of size 1, including the key dim, which is expanded."""
    import torch
    from vidax_amd.attention import _full_bias, _key_only
    B, H, Sq, Sk = 2, 3, 5, 70
    for shape in [(1, H, Sq, 1), (B, 1, Sq, 1), (B, H, Sq, Sk), (H, Sq, Sk), (Sq, 1), (1, 1, 1, Sk)]:
        x = torch.randn(shape)
        fb, strides = _full_bias(x, B, H, Sq, Sk, "cpu")
        assert fb.shape[3] == 128 and fb.dtype == torch.float32
        full = torch.broadcast_to(x.reshape((1,) * (4 - x.dim()) + tuple(shape)), (B, H, Sq, Sk))
        for b in range(B):
            for h in range(H):
                for q in range(Sq):
                    row = fb.flatten()[b * strides[0] + h * strides[1] + q * strides[2]:][:Sk]
                    assert torch.equal(row, full[b, h, q]), shape
    with pytest.raises(ValueError):
        _full_bias(torch.zeros(1, H, Sq, 7), B, H, Sq, Sk, "cpu")
    m = torch.tensor([True, False]).reshape(2, 1, 1, 1)
    assert torch.equal(_key_only(m, B, Sk, "mask"), m.reshape(2, 1).expand(2, Sk))
    assert _key_only(torch.zeros(1, 1, Sq, 1), B, Sk, "bias") is None


def test_na3d_inputs_are_realigned():
    """A contiguous view at an address that is not 16-byte aligned is copied
    for the kernel; aligned contiguous tensors are passed as they are."""
    import torch
    from vidax_amd.natten import _aligned16
    buf = torch.zeros(4096, dtype=torch.bfloat16)
    view = buf[3:3 + 2 * 4 * 8].view(1, 1, 1, 2, 4, 8)
    assert view.data_ptr() % 16 != 0
    fixed = _aligned16(view)
    assert fixed.data_ptr() % 16 == 0 and torch.equal(fixed, view)
    good = buf[8:8 + 64].view(1, 1, 1, 2, 4, 8)
    assert _aligned16(good) is good


def _qprep_check(**kw):
    args = dict(q=A, w=A, eps=1e-6, post=0.125, cos=A, sin=A, stride=64, D=128, kw=7)
    args.update(kw)
    return _lib.lib().vx_na3d_qprep_check(args["q"], A, A, A, 1, 3, 8, 80, 2, args["D"], 3, 7, args["kw"],
                                          args["w"], ctypes.c_float(args["eps"]), ctypes.c_float(args["post"]),
                                          args["cos"], args["sin"], args["stride"])


def test_na3d_qprep_check():
    assert _qprep_check() == _lib.VX_OK
    assert _qprep_check(w=None, cos=None, sin=None, post=1.0) == _lib.VX_OK   # plain NA
    assert _qprep_check(D=64, stride=32) == _lib.VX_OK
    for kw, code, frag in [
        (dict(w=A + 4), _lib.VX_ERR_INVALID_ARGUMENT, "q_norm_weight"),
        (dict(eps=-1.0), _lib.VX_ERR_INVALID_ARGUMENT, "eps"),
        (dict(post=float("nan")), _lib.VX_ERR_INVALID_ARGUMENT, "q_post_scale"),
        (dict(sin=None), _lib.VX_ERR_INVALID_ARGUMENT, "both"),
        (dict(cos=A + 8), _lib.VX_ERR_INVALID_ARGUMENT, "aligned"),
        (dict(stride=62), _lib.VX_ERR_INVALID_ARGUMENT, "rope_stride"),
        (dict(stride=60), _lib.VX_ERR_INVALID_ARGUMENT, "rope_stride"),
        (dict(q=None), _lib.VX_ERR_INVALID_ARGUMENT, "non-NULL"),
    ]:
        assert _qprep_check(**kw) == code, kw
        assert frag in _lib.last_error(), (kw, _lib.last_error())


def _axes_check(q=A, D=128, split=(32, 48, 48), stride=64, cos=A, sin=A, grid=(3, 8, 80), post=0.088):
    sp = None if split is None else (ctypes.c_int32 * 3)(*split)
    return _lib.lib().vx_na3d_qprep_axes_check(q, A, A, A, 1, *grid, 2, D, 3, 7, 7, A, ctypes.c_float(1e-6),
                                               ctypes.c_float(post), cos, sin, stride, sp)


def test_na3d_qprep_axes_check():
    """The per-axis rope rows: split even and summing to head_dim, t and h
    parts multiples of 8, aligned tables of whole 16-byte rows of at least
    head_dim/2 floats, (t + h + w) rows addressable with 32-bit offsets."""
    assert _axes_check() == _lib.VX_OK
    assert _axes_check(D=64, split=(16, 24, 24), stride=32) == _lib.VX_OK
    assert _axes_check(split=(0, 64, 64), stride=68) == _lib.VX_OK
    assert _axes_check(split=None, cos=None, sin=None) == _lib.VX_OK  # no rope
    for kw, code, frag in [
        (dict(split=(32, 48, 40)), _lib.VX_ERR_INVALID_ARGUMENT, "sum to head_dim"),
        (dict(split=(33, 47, 48)), _lib.VX_ERR_INVALID_ARGUMENT, "even"),
        (dict(split=(36, 44, 48)), _lib.VX_ERR_UNSUPPORTED, "multiples of 8"),
        (dict(stride=60), _lib.VX_ERR_INVALID_ARGUMENT, "rope_stride"),
        (dict(stride=66), _lib.VX_ERR_INVALID_ARGUMENT, "rope_stride"),
        (dict(split=None), _lib.VX_ERR_INVALID_ARGUMENT, "rope_split"),
        (dict(sin=None), _lib.VX_ERR_INVALID_ARGUMENT, "both"),
        (dict(cos=A + 8), _lib.VX_ERR_INVALID_ARGUMENT, "aligned"),
        (dict(grid=(3, 8, 80), stride=(1 << 31) // 91 + 4 & ~3), _lib.VX_ERR_UNSUPPORTED, "2^31"),
        (dict(q=None), _lib.VX_ERR_INVALID_ARGUMENT, "non-NULL"),
    ]:
        assert _axes_check(**kw) == code, kw
        assert frag in _lib.last_error(), (kw, _lib.last_error())


def _split(shape, cus=256):
    a, b, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    rc = _lib.lib().vx_flash_attn_split_plan(*shape, cus, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    assert rc == _lib.VX_OK
    return a.value, b.value, c.value


def test_flash_split_plan():
    """Key split of a grid's last round: only when that round holds at most
    half the resident workgroups and the keys span >= 16 tiles; the workspace
    holds two fp32 partials (O, reference point, row sum per lane) per item."""
    # c1: 61 x 12 = 732 items of 128 queries over 2 x 256 slots: 220 split at tile 61
    assert _split((1, 7800, 7800, 12, 128)) == (220, 61 * 64, 2 * 220 * 4 * 64 * (4 * 16 + 2) * 4)
    assert _split((1, 32760, 32760, 40, 128)) == (0, 0, 0)     # 5120 items: whole waves of workgroups
    assert _split((2, 32760, 512, 40, 128)) == (0, 0, 0)       # short keys
    assert _split((1, 119056, 119056, 24, 128)) == (0, 0, 0)   # last wave of workgroups: 176 > 128 of 256
    assert _split((1, 2048, 1500, 3, 128)) == (48, 768, 2 * 48 * 4 * 64 * 66 * 4)
    assert _split((1, 8192, 2048, 25, 128))[0] == 32            # 8-wave: 800 items, 256 slots
    assert _split((1, 8192, 2048, 25, 64))[2] == 2 * 32 * 8 * 64 * (2 * 16 + 2) * 4
    assert _split((1, 7800, 7800, 12, 128), cus=0) == (0, 0, 0)
    assert _split((1, 7800, 900, 12, 128)) == (0, 0, 0)        # 15 key tiles


def test_ws_fwd_rejects_before_launch():
    L = _lib.lib()
    args = [A, A, A, A, None, None, None, 0, 1, 100, 200, 4, 128, None, None, None, None, ctypes.c_float(0.1)]
    assert L.vx_flash_attn_ws_fwd(*args, A + 8, 1024, None) == _lib.VX_ERR_INVALID_ARGUMENT
    assert "workspace" in _lib.last_error()
    assert L.vx_flash_attn_ws_fwd(*args, A, -1, None) == _lib.VX_ERR_INVALID_ARGUMENT
    args[12] = 96
    assert L.vx_flash_attn_ws_fwd(*args, A, 1024, None) == _lib.VX_ERR_UNSUPPORTED


@pytest.mark.parametrize("D,code", [(64, _lib.VX_OK), (128, _lib.VX_OK),
                                    (80, _lib.VX_ERR_UNSUPPORTED), (384, _lib.VX_ERR_UNSUPPORTED)])
def test_flash_head_dim_check_for_drop_in_branch(D, code):
    """The trace-time check a drop-in branch makes before choosing the kernel:
    CLIP vision runs dot_product_attention at D=80 (16 heads of dim 1280,
    wan/wan2_1/clip_vision.py:36-46) and the Wan2.1 VAE's middle attention at
    one head of D=384 (wan/common/vae_layers.py:100-110); both keep the
    reference's jax.nn path. The check is host-only (no GPU)."""
    import vidax_amd
    from vidax_amd.attention import _require_supported
    # CLIP: 257 tokens x 16 heads; VAE middle block: one 60x104 frame, 1 head
    B, S, H = (1, 257, 16) if D == 80 else (1, 6240, 1) if D == 384 else (1, 4096, 8)
    assert _flash_check(B=B, Sq=S, Sk=S, H=H, D=D) == code
    if code == _lib.VX_ERR_UNSUPPORTED:
        assert "head_dim" in _lib.last_error()
    assert vidax_amd.flash_supported(B, S, S, H, D) == (code == _lib.VX_OK)
    assert _lib.flash_shape_check(B, S, S, H, D)[0] == code
    if code == _lib.VX_OK:
        _require_supported(B, S, S, H, D)
    else:
        with pytest.raises(NotImplementedError, match=rf"head_dim {D} .*jax\.nn\.dot_product_attention.*flash_supported"):
            _require_supported(B, S, S, H, D)


def test_flash_kernel_name_with_the_key_split():
    """With the device's compute-unit count the name follows the workspace
    entry point that flash_attention calls: the key-split kernel for grids
    whose last round would leave most of the device idle, never with a key
    or full bias (those never split)."""
    from vidax_amd.attention import flash_kernel_name
    assert flash_kernel_name(1, 7800, 7800, 12) == "flash_fwd_kernel<0, 128, 4>"
    assert flash_kernel_name(1, 7800, 7800, 12, num_cus=256) == "flash_fwd_split_kernel<0, 128, 4>"
    assert flash_kernel_name(1, 7800, 7800, 12, 128, 1, num_cus=256) == "flash_fwd_split_kernel<1, 128, 4>"
    assert flash_kernel_name(1, 7800, 7800, 12, 128, 2, num_cus=256) == "flash_fwd_kernel<2, 128, 4>"
    assert flash_kernel_name(1, 32760, 32760, 40, num_cus=256) == "flash_fwd_kernel<0, 128, 8>"   # 5120 tiles
    assert flash_kernel_name(2, 32760, 512, 40, num_cus=256) == "flash_stream_kernel<128>"
