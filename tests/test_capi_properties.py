"""Property tests of the C ABI's host side (CPU, no kernel launch): random
sizes, strides and pointers, valid or not, through the argument checks and
the launch-plan queries. Every call must return one of the documented codes
(never crash), leave a message exactly when it fails, and agree with the
rules the header states; the neighbourhood plan is compared with the rule
written out here on its own (x window, grid height and width, t window)."""
import ctypes

import pytest

from vidax_amd import _lib

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402

A = 1 << 20  # a 16-byte aligned fake device address (never dereferenced)
CODES = {_lib.VX_OK, _lib.VX_ERR_INVALID_ARGUMENT, _lib.VX_ERR_UNSUPPORTED}
SETTINGS = settings(max_examples=400, deadline=None, suppress_health_check=[HealthCheck.too_slow])

# Each field is valid most of the time, so that both accepted and rejected
# calls are drawn often.
sizes = st.one_of(st.integers(1, 70000), st.integers(1, 70000), st.integers(1, 70000), st.integers(1, 70000),
                  st.integers(-3, 0), st.sampled_from([2 ** 31 - 1, -2 ** 31]))
small = st.one_of(st.integers(1, 64), st.integers(1, 64), st.integers(1, 64), st.integers(-3, 0))
ptrs = st.sampled_from([A] * 12 + [None, A + 8, A + 4, A + 1])


_SEEN = {"flash": set(), "na3d": set()}  # return codes drawn, per checker


def _s3(s):
    return None if s is None else _lib.strides3(s)


@SETTINGS
@given(B=small, Sq=sizes, Sk=sizes, H=small, D=st.sampled_from([64, 128] * 6 + [0, 32, 80, 96, 256, 384]),
       q=ptrs, k=ptrs, v=ptrs, out=ptrs, kv_len=st.sampled_from([None, None, A, A + 2]),
       key_valid=st.sampled_from([None] * 4 + [A, A, A + 2]), key_bias=st.sampled_from([None] * 4 + [A, A, A + 4]),
       stride=st.one_of(st.integers(70016, 80000), st.integers(-8, 80000)),
       scale=st.sampled_from([0.088] * 8 + [1.0, 0.0, -1.0, 1e-40, float("inf"), float("nan")]),
       qs=st.one_of(st.none(), st.none(), st.tuples(st.integers(-5, 2 ** 34), st.integers(-5, 2 ** 26),
                                                    st.integers(-5, 2 ** 12))))
def test_flash_check_never_fails_silently(B, Sq, Sk, H, D, q, k, v, out, kv_len, key_valid, key_bias, stride, scale, qs):
    rc = _lib.lib().vx_flash_attn_check(q, k, v, out, kv_len, key_valid, key_bias, stride, B, Sq, Sk, H, D,
                                        _s3(qs), None, None, None, ctypes.c_float(scale))
    assert rc in CODES
    _SEEN["flash"].add(rc)
    msg = _lib.last_error()
    assert (rc == _lib.VX_OK) == (msg == ""), (rc, msg)
    if rc == _lib.VX_OK:
        # what the header promises of an accepted call
        assert None not in (q, k, v, out) and all(p % 16 == 0 for p in (q, k, v, out))
        assert B >= 1 and Sq >= 1 and Sk >= 1 and H >= 1 and D in (64, 128)
        assert scale > 0 and scale != float("inf")
        if key_valid is not None or key_bias is not None:
            assert stride >= (Sk + 63) // 64 * 64 and stride % 4 == 0
        # the launch plan of an accepted shape names a kernel
        mask = (1 if key_valid is not None else 0) | (2 if key_bias is not None else 0)
        name = _lib.flash_plan(B, Sq, Sk, H, D, mask)
        assert name.startswith("flash_") and f", {D}" in name


def _na_rule(T, H, W, D, kt, kw):
    """The neighbourhood kernel for a grid and window, from the rule as the
    header and the design state it (clamped windows kt' = min(kt, T), kw' =
    min(kw, W))."""
    k, t = min(kw, W), min(kt, T)
    up = lambda n, m: -(-n // m) * m
    if k <= 9:
        if D == 64 and up(H, 8) * up(W, 16) <= up(H, 4) * up(W, 32):
            return "na3d_tall_kernel<64>"
        if D == 128 and t >= 2:
            return "na3d_tstack_kernel<128>"
        return f"na3d_pipe_kernel<16, {D}>"
    if k <= 13:
        if D == 64 and up(W, 32) == up(W, 16):
            return "na3d_deep_kernel<64>" if t >= 5 else "na3d_tall_wide_kernel<64>"
        return f"na3d_tall_kernel<{D}>"
    if k <= 25:
        return f"na3d_pipe_kernel<32, {D}>"
    return f"na3d_wave_kernel<{D}>"


@SETTINGS
@given(T=st.integers(1, 64), H=st.integers(1, 200), W=st.integers(1, 400), D=st.sampled_from([64, 128]),
       kt=st.integers(1, 40), kh=st.integers(1, 40), kw=st.integers(1, 130))
def test_na3d_plan_follows_the_rule(T, H, W, D, kt, kh, kw):
    assert _lib.na3d_plan(T, H, W, D, kt, kh, kw) == _na_rule(T, H, W, D, kt, kw)


@SETTINGS
@given(B=small, T=small, H=st.one_of(small, sizes), W=st.one_of(small, sizes), NH=small,
       D=st.sampled_from([64, 128] * 6 + [0, 32, 96, 256]),
       kt=st.integers(-2, 50), kh=st.integers(-2, 50), kw=st.integers(-2, 300), q=ptrs, out=ptrs,
       scale=st.sampled_from([1.0] * 6 + [0.125, 0.0, float("nan"), -2.0]))
def test_na3d_check_never_fails_silently(B, T, H, W, NH, D, kt, kh, kw, q, out, scale):
    rc = _lib.lib().vx_na3d_check(q, A, A, out, B, T, H, W, NH, D, kt, kh, kw, ctypes.c_float(scale))
    assert rc in CODES
    _SEEN["na3d"].add(rc)
    assert (rc == _lib.VX_OK) == (_lib.last_error() == "")
    if rc == _lib.VX_OK:
        assert q is not None and out is not None and q % 16 == 0 and out % 16 == 0
        assert min(B, T, H, W, NH, kt, kh, kw) >= 1 and D in (64, 128) and scale > 0
        assert W * NH * D < 2 ** 30


def test_both_outcomes_were_drawn():
    """The draws above reached both accepted and rejected calls (run after
    them: pytest keeps a module's order)."""
    for name in ("flash", "na3d"):
        if not _SEEN[name]:
            pytest.skip("run together with the property tests above")
        assert _lib.VX_OK in _SEEN[name] and len(_SEEN[name]) >= 2, (name, _SEEN[name])
