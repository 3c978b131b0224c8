"""Attention prologue (q/k RMSNorm + 3D rotary embedding).

CPU: the oracle (oracle/prologue_oracle.py) is pinned by an independent
library routine (torch's rms_norm in fp32), known answers, the algebra of
rotations (identity at position 0, norm preservation, inverse, translation
invariance of q.k), the T/H/W frequency split, and planted mistakes.
GPU: the HIP kernel (through vx_rmsnorm_rope_fwd) against the oracle: every
element within one bf16 ulp of the oracle and at least 99% bit-identical
(the oracle's fp32 mean-of-squares, rsqrt and cos/sin may differ from the
kernel's in the last fp32 bit, which can move a bf16 rounding by one ulp).
"""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as A
from oracle import prologue_oracle as P

ULP_TOL = 1.0       # bf16 ulps
EXACT_FRAC = 0.99   # fraction of bit-identical elements


def _bf16_normal(rng, shape, scale=1.0):
    return A.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


# ------------------------------------------------------------------ oracle
def test_rms_norm_matches_torch_fp32():
    """Formula (mean of squares over the last axis, eps inside the rsqrt,
    weight per channel) against torch's rms_norm, with no bf16 rounding."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5, 256)).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (256,), torch.from_numpy(w).double(), eps=1e-6)
    var = np.mean(np.square(x.astype(np.float64)), axis=-1, keepdims=True)
    mine = x.astype(np.float64) / np.sqrt(var + 1e-6) * w
    np.testing.assert_allclose(mine, ref.numpy(), rtol=1e-12, atol=1e-12)
    # the oracle is this formula with the reference's two bf16 roundings
    y = P.rms_norm(A.bf16_round(x), np.ones(256, np.float32))
    x64 = A.bf16_round(x).astype(np.float64)
    exact = x64 / np.sqrt(np.mean(x64 ** 2, axis=-1, keepdims=True) + 1e-6)
    assert np.max(np.abs(y - exact) / (np.abs(exact) + 1e-30)) < 2 ** -7


def test_rms_norm_known_answers():
    # constant rows normalise to 1 (1/sqrt(1 + 1e-6) rounds to 1 in bf16): out = bf16(w)
    w = np.array([0.5, -3.0, 1.0 / 3.0, 7.1], np.float32)
    out = P.rms_norm(np.full((2, 4), 2.5, np.float32), w)
    np.testing.assert_array_equal(out, np.broadcast_to(A.bf16_round(w), (2, 4)))
    # [3, 4]: mean square 12.5 -> x / sqrt(12.5) = [0.8485.., 1.1313..] -> bf16
    out = P.rms_norm(np.array([[3.0, 4.0]], np.float32), np.ones(2, np.float32), eps=0.0)
    np.testing.assert_array_equal(out, [[0.84765625, 1.1328125]])


def test_rope_tables_split_and_frequencies():
    """Pairs 0..21 follow t, 22..42 follow h, 43..63 follow w (head_dim 128),
    and pair j of an axis with d pairs turns by pos * theta^(-j/d)."""
    T, H, W = 3, 4, 5
    cos, sin = P.create_rope3d_freqs(T, H, W, 128)
    assert cos.shape == (T * H * W, 64)
    ang = np.arctan2(sin, cos).reshape(T, H, W, 64)
    vary_t = np.abs(np.diff(ang, axis=0)).max(axis=(0, 1, 2)) > 0
    vary_h = np.abs(np.diff(ang, axis=1)).max(axis=(0, 1, 2)) > 0
    vary_w = np.abs(np.diff(ang, axis=2)).max(axis=(0, 1, 2)) > 0
    assert vary_t.tolist() == [True] * 22 + [False] * 42
    assert vary_h.tolist() == [False] * 22 + [True] * 21 + [False] * 21
    assert vary_w.tolist() == [False] * 43 + [True] * 21
    for base, d, axis_pos in ((0, 22, (1, 0, 0)), (22, 21, (0, 1, 0)), (43, 21, (0, 0, 1))):
        pos = np.ravel_multi_index(axis_pos, (T, H, W))
        j = np.arange(d)
        np.testing.assert_allclose(ang[np.unravel_index(pos, (T, H, W))][base:base + d],
                                   10000.0 ** (-j / d), rtol=2e-6)


def test_rope_rotation_algebra():
    rng = np.random.default_rng(1)
    T, H, W, D = 2, 3, 4, 128
    S = T * H * W
    cos, sin = P.create_rope3d_freqs(T, H, W, D)
    x = _bf16_normal(rng, (1, S, 2, D))
    y = P.apply_rope3d(x, cos, sin)
    # position 0 is the identity
    np.testing.assert_array_equal(y[:, 0], x[:, 0])
    # pair norms are preserved (to bf16 rounding)
    n_in = np.hypot(x[..., 0::2], x[..., 1::2])
    n_out = np.hypot(y[..., 0::2], y[..., 1::2])
    assert np.max(np.abs(n_out - n_in) / (n_in + 1e-3)) < 2 ** -6
    # rotating back by the opposite angle recovers the input
    back = P.apply_rope3d(y, cos, -sin)
    assert np.max(np.abs(back - x)) < 2 ** -5 * np.max(np.abs(x))


def test_rope_translation_invariance():
    """q.k after rotation depends on the position difference only (pins
    angles linear in position with one angle per pair for q and k)."""
    rng = np.random.default_rng(2)
    W = 40
    cos, sin = P.create_rope3d_freqs(1, 1, W, 128)
    q = rng.standard_normal(128)
    k = rng.standard_normal(128)

    def rot(v, pos):  # float64, no rounding
        c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
        v1, v2 = v[0::2], v[1::2]
        out = np.empty(128)
        out[0::2] = v1 * c - v2 * s
        out[1::2] = v2 * c + v1 * s
        return out

    d1 = rot(q, 7) @ rot(k, 3)
    d2 = rot(q, 30) @ rot(k, 26)
    d3 = rot(q, 12) @ rot(k, 3)
    assert abs(d1 - d2) < 1e-3 * (abs(d1) + 1)
    assert abs(d1 - d3) > 1e-3  # a different offset gives a different product


def test_planted_mistakes_are_caught():
    cos, sin = P.create_rope3d_freqs(6, 1, 1, 128)  # positions along t: pair 0 turns
    x = np.zeros((1, 6, 1, 128), np.float32)
    x[..., 0] = 1.0  # unit vector on pair 0
    y = P.apply_rope3d(x, cos, sin)
    # adjacent-pair convention: only entries 0 and 1 move
    assert np.all(y[..., 2:] == 0) and np.any(y[..., 1] != 0)
    # a rotate-half implementation would write entry 64 instead of 1
    half = np.concatenate([x[..., :64] * cos[None, :, None, :] , x[..., :64] * sin[None, :, None, :]], axis=-1)
    assert not np.allclose(half, y)
    # a norm with sum instead of mean is caught by the known answer above
    xx = np.array([[3.0, 4.0]], np.float32)
    wrong = A.bf16_round(A.bf16_round(xx / np.sqrt(np.sum(xx ** 2) + 0.0)))
    assert not np.array_equal(wrong, P.rms_norm(xx, np.ones(2, np.float32), eps=0.0))


# ------------------------------------------- neighbourhood block (abs RoPE)
def test_abs_rope_split_known_answers():
    """(d_t, d_h, d_w): head_dim 40 takes the odd-half branch (d_t 10 -> 8)."""
    assert P.default_rope_dim_split(64) == (16, 24, 24)
    assert P.default_rope_dim_split(128) == (32, 48, 48)
    assert P.default_rope_dim_split(96) == (24, 36, 36)
    assert P.default_rope_dim_split(40) == (8, 16, 16)
    assert P.default_rope_dim_split(32) == (8, 12, 12)


def _complex_rotation(x, split, base=10000.0):
    """float64 rotation written as complex multiplication: the pair
    (x[2j], x[2j+1]) of axis chunk a is the number x[2j] + i x[2j+1], times
    exp(i * pos_a * base^(-2j/d_a))."""
    _, T, H, W, _, HD = x.shape
    out = np.empty(x.shape, np.float64)
    lo = 0
    for axis, (d, n) in enumerate(zip(split, (T, H, W))):
        z = x[..., lo:lo + d:2].astype(np.float64) + 1j * x[..., lo + 1:lo + d:2]
        theta = np.arange(n)[:, None] * base ** (-np.arange(0, d, 2) / d)[None, :]
        shape = [1, 1, 1, 1, 1, d // 2]
        shape[axis + 1] = n
        z = z * np.exp(1j * theta.reshape(shape))
        out[..., lo:lo + d:2], out[..., lo + 1:lo + d:2] = z.real, z.imag
        lo += d
    return out


@pytest.mark.parametrize("HD", [64, 128, 40])
def test_abs_rope_matches_complex_rotation(HD):
    """Pins the interleaved pairing, the sign of the rotation, the frequency
    formula and which channels follow T, H and W."""
    rng = np.random.default_rng(HD)
    x = _bf16_normal(rng, (1, 3, 4, 5, 2, HD))
    got = P.apply_abs_rope3d(x)
    ref = _complex_rotation(x, P.default_rope_dim_split(HD))
    assert np.max(np.abs(got - ref)) <= 2 ** -8 * np.max(np.abs(ref)) + 1e-6
    # mistakes that must fail the same check
    split = P.default_rope_dim_split(HD)
    wrong_axes = _complex_rotation(x, split[::-1]) if split[0] != split[2] else None
    if wrong_axes is not None:
        assert np.max(np.abs(got - wrong_axes)) > 1e-2
    neg = _complex_rotation(x[..., :], split)
    neg[..., 1::2] = -_complex_rotation(x * np.where(np.arange(HD) % 2, -1, 1), split)[..., 1::2]
    assert np.max(np.abs(got - neg)) > 1e-2  # the conjugate rotation


def test_abs_rope_tables_equal_axis_form():
    """The per-token tables (the kernel's input) applied pair by pair give
    the same bits as the axis-by-axis form."""
    rng = np.random.default_rng(5)
    T, H, W, NH, HD = 3, 4, 6, 3, 64
    x = _bf16_normal(rng, (2, T, H, W, NH, HD))
    cos, sin = P.create_abs_rope3d_freqs(T, H, W, HD)
    via_tables = P.apply_rope3d(x.reshape(2, T * H * W, NH, HD), cos, sin).reshape(x.shape)
    np.testing.assert_array_equal(via_tables, P.apply_abs_rope3d(x))
    # the origin token is not rotated; along W only the last 12 pairs turn
    np.testing.assert_array_equal(cos[0], 1.0)
    moved = np.abs(np.arctan2(sin, cos).reshape(T, H, W, 32)[0, 0, 1]) > 0
    assert moved.tolist() == [False] * 20 + [True] * 12


def test_abs_rope_axis_tables_equal_token_tables():
    """The per-axis rows the fused NA kernel reads (t rows, then h rows, then
    w rows, each axis in its own pair columns), gathered per token as the
    kernel reads them, are bit for bit the per-token tables (both come from
    one per-axis routine)."""
    from vidax_amd import create_abs_rope3d_axis_freqs, create_abs_rope3d_freqs
    for T, H, W, HD, split in [(3, 5, 7, 64, None), (2, 4, 6, 128, None), (4, 3, 5, 64, (16, 24, 24)),
                               (2, 3, 4, 128, (0, 64, 64)), (1, 2, 3, 64, (32, 32, 0))]:
        cos, sin = create_abs_rope3d_freqs(T, H, W, HD, rope_split=split)
        ax = create_abs_rope3d_axis_freqs(T, H, W, HD, rope_split=split)
        p_t, p_h = ax.split[0] // 2, (ax.split[0] + ax.split[1]) // 2
        assert ax.grid == (T, H, W) and sum(ax.split) == HD
        assert ax.cos.shape == (T + H + W, -(-(HD // 2) // 4) * 4) and ax.cos.dtype == torch.float32
        t, y, x = torch.meshgrid(torch.arange(T), torch.arange(H), torch.arange(W), indexing="ij")
        j = torch.arange(HD // 2)
        row = torch.where(j < p_t, t[..., None], torch.where(j < p_h, T + y[..., None], T + H + x[..., None]))
        for tok, tab in ((cos, ax.cos), (sin, ax.sin)):
            gathered = tab[row, j.expand_as(row)]
            assert torch.equal(gathered.reshape(tok.shape), tok)


def test_abs_rope_relative_positions():
    """q.k after rotation depends only on the offset along each axis."""
    rng = np.random.default_rng(6)
    T, H, W, HD = 5, 6, 7, 64
    q = rng.standard_normal(HD)
    k = rng.standard_normal(HD)
    cos, sin = P.create_abs_rope3d_freqs(T, H, W, HD)

    def rot(v, t, h, w):
        i = (t * H + h) * W + w
        c, s = cos[i].astype(np.float64), sin[i].astype(np.float64)
        out = np.empty(HD)
        out[0::2] = v[0::2] * c - v[1::2] * s
        out[1::2] = v[0::2] * s + v[1::2] * c
        return out

    base = rot(q, 2, 3, 4) @ rot(k, 1, 1, 2)
    assert abs(base - rot(q, 4, 5, 6) @ rot(k, 3, 3, 4)) < 1e-6 * (abs(base) + 1)  # fp32 tables
    assert abs(base - rot(q, 2, 3, 5) @ rot(k, 1, 1, 2)) > 1e-4


def test_post_scale_known_answers():
    """q * head_dim^-0.5 in bf16: the scalar is rounded to bf16 first
    (128^-0.5 -> 0.08837890625); 64^-0.5 = 0.125 is exact."""
    y = np.array([[1.0, 3.0, -0.5, 1.5]], np.float32).reshape(1, 1, 1, 1, 1, 4)
    out = P.na3d_qk_norm_rope(y, None, post_scale=128 ** -0.5, rope=False)
    np.testing.assert_array_equal(out.ravel(), A.bf16_round(y.ravel() * np.float32(0.08837890625)))
    assert A.bf16_round(np.float32(128 ** -0.5)) == np.float32(0.08837890625)
    out = P.na3d_qk_norm_rope(y, None, post_scale=0.125, rope=False)
    np.testing.assert_array_equal(out.ravel(), y.ravel() / 8)


# ------------------------------------------------------------------ GPU
def _ulps(got, ref):
    ref = np.asarray(ref, np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    return np.abs(np.asarray(got, np.float64) - ref) / ulp


def _check(got, ref, label):
    u = _ulps(got, ref)
    frac = float(np.mean(u == 0))
    print(f"  {label}: max_ulps={u.max():.1f} exact={frac:.5f}", flush=True)
    assert np.isfinite(got).all(), label
    assert u.max() <= ULP_TOL and frac >= EXACT_FRAC, label


def _dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu).to(torch.bfloat16)


PROLOGUE_CASES = [
    # (B, (T, Hg, Wg), H, D, norm, rope)
    (2, (2, 3, 5), 4, 128, True, True),
    (1, (3, 4, 6), 40, 128, True, True),   # Wan2.1-14B row: 40 heads x 128
    (1, (1, 5, 7), 12, 128, True, False),
    (2, (2, 2, 9), 8, 128, False, True),
    (1, (2, 3, 4), 6, 64, True, True),     # head_dim 64
    (1, (1, 2, 33), 64, 128, True, True),  # widest row: 8192
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,grid,H,D,norm,rope", PROLOGUE_CASES)
def test_qk_norm_rope_matches_oracle(gpu, B, grid, H, D, norm, rope):
    from vidax_amd import create_rope3d_freqs, qk_norm_rope
    print(f"[case] qk_norm_rope B={B} grid={grid} H={H} D={D} norm={norm} rope={rope}", flush=True)
    rng = np.random.default_rng(sum(grid) + H + D)
    S = int(np.prod(grid))
    x = _bf16_normal(rng, (B, S, H * D), 3.0)
    w = (1.0 + 0.5 * rng.standard_normal(H * D)).astype(np.float32) if norm else None
    cos, sin = P.create_rope3d_freqs(*grid, D) if rope else (None, None)
    ref = P.qk_norm_rope(x, w, cos, sin, H)
    freqs = create_rope3d_freqs(*grid, D, device=gpu) if rope else None
    out = qk_norm_rope(_dev(x, gpu), torch.from_numpy(w).to(gpu) if norm else None, freqs, H)
    torch.cuda.synchronize()
    _check(out.float().cpu().numpy(), ref, "qk_norm_rope")


@pytest.mark.gpu
def test_rope_tables_match_oracle(gpu):
    from vidax_amd import create_rope3d_freqs
    cos, sin = create_rope3d_freqs(4, 6, 9, 128, device=gpu)
    rc, rs = P.create_rope3d_freqs(4, 6, 9, 128)
    np.testing.assert_allclose(cos.reshape(-1, 64).cpu().numpy(), rc, atol=2e-6)
    np.testing.assert_allclose(sin.reshape(-1, 64).cpu().numpy(), rs, atol=2e-6)


@pytest.mark.gpu
def test_per_head_rms_norm_and_rope_separately(gpu):
    from vidax_amd import apply_rope3d, rms_norm
    print("[case] per-head rms_norm, then apply_rope3d", flush=True)
    rng = np.random.default_rng(9)
    B, S, H, D = 2, 24, 6, 128
    x = _bf16_normal(rng, (B, S, H, D), 2.0)
    w = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
    y = rms_norm(_dev(x, gpu), torch.from_numpy(w).to(gpu))
    torch.cuda.synchronize()
    _check(y.float().cpu().numpy(), P.rms_norm(x, w), "per-head rms_norm")
    cos, sin = P.create_rope3d_freqs(2, 3, 4, D)
    z = apply_rope3d(y, (torch.from_numpy(cos).to(gpu), torch.from_numpy(sin).to(gpu)))
    torch.cuda.synchronize()
    _check(z.float().cpu().numpy(), P.apply_rope3d(y.float().cpu().numpy(), cos, sin), "apply_rope3d")


@pytest.mark.gpu
def test_whole_row_rms_norm_3d_input(gpu):
    from vidax_amd import rms_norm
    rng = np.random.default_rng(10)
    x = _bf16_normal(rng, (3, 17, 1536), 0.7)
    w = rng.standard_normal(1536).astype(np.float32)
    y = rms_norm(_dev(x, gpu), torch.from_numpy(w).to(gpu))
    torch.cuda.synchronize()
    _check(y.float().cpu().numpy(), P.rms_norm(x, w), "row rms_norm")


@pytest.mark.gpu
def test_strided_rows_from_fused_qkv(gpu):
    """q as a slice of a fused (B, S, 3 * H * D) projection: no copy needed."""
    from vidax_amd import create_rope3d_freqs, qk_norm_rope
    rng = np.random.default_rng(11)
    B, grid, H, D = 2, (2, 3, 3), 4, 128
    S = 18
    qkv = _bf16_normal(rng, (B, S, 3 * H * D))
    w = rng.standard_normal(H * D).astype(np.float32)
    t = _dev(qkv, gpu)
    out = qk_norm_rope(t[..., H * D:2 * H * D], torch.from_numpy(w).to(gpu),
                       create_rope3d_freqs(*grid, D, device=gpu), H)
    torch.cuda.synchronize()
    cos, sin = P.create_rope3d_freqs(*grid, D)
    _check(out.float().cpu().numpy(), P.qk_norm_rope(qkv[..., H * D:2 * H * D], w, cos, sin, H), "k slice")


@pytest.mark.gpu
def test_unsupported_rows_raise(gpu):
    from vidax_amd import qk_norm_rope
    x = torch.zeros((1, 4, 72 * 128), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(NotImplementedError):
        qk_norm_rope(x, None, None, 72)


NA_PROLOGUE_CASES = [
    # (B, (T, H, W), NH, HD, norm, post_scale, rope)
    (1, (3, 5, 7), 4, 64, True, 64 ** -0.5, True),     # LTX-2.5 q: head_dim 64
    (2, (2, 4, 6), 4, 64, True, 1.0, True),            # k: no scale
    (1, (3, 4, 9), 8, 128, True, 128 ** -0.5, True),   # head_dim 128
    (1, (2, 3, 5), 6, 64, False, 1.0, True),           # rope only
    (1, (2, 3, 5), 2, 128, True, 0.7, False),          # norm and scale only
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,grid,NH,HD,norm,post,rope", NA_PROLOGUE_CASES)
def test_na3d_qk_norm_rope_matches_oracle(gpu, B, grid, NH, HD, norm, post, rope):
    from vidax_amd import create_abs_rope3d_freqs, na3d_qk_norm_rope
    print(f"[case] na3d_qk_norm_rope B={B} grid={grid} NH={NH} HD={HD} norm={norm} post={post:.4f} rope={rope}",
          flush=True)
    rng = np.random.default_rng(sum(grid) * NH + HD)
    x = _bf16_normal(rng, (B, *grid, NH, HD), 2.0)
    w = (1.0 + 0.5 * rng.standard_normal(HD)).astype(np.float32) if norm else None
    ref = P.na3d_qk_norm_rope(x, w, post_scale=post, rope=rope)
    freqs = create_abs_rope3d_freqs(*grid, HD, device=gpu) if rope else None
    out = na3d_qk_norm_rope(_dev(x, gpu), torch.from_numpy(w).to(gpu) if norm else None, freqs, post_scale=post)
    torch.cuda.synchronize()
    _check(out.float().cpu().numpy(), ref, "na3d_qk_norm_rope")


@pytest.mark.gpu
def test_abs_rope_tables_and_apply_match_oracle(gpu):
    from vidax_amd import apply_abs_rope3d, create_abs_rope3d_freqs
    cos, sin = create_abs_rope3d_freqs(4, 6, 9, 64, device=gpu)
    rc, rs = P.create_abs_rope3d_freqs(4, 6, 9, 64)
    np.testing.assert_allclose(cos.reshape(-1, 32).cpu().numpy(), rc, atol=2e-6)
    np.testing.assert_allclose(sin.reshape(-1, 32).cpu().numpy(), rs, atol=2e-6)
    rng = np.random.default_rng(12)
    x = _bf16_normal(rng, (1, 4, 6, 9, 3, 64))
    out = apply_abs_rope3d(_dev(x, gpu), (cos, sin))
    torch.cuda.synchronize()
    _check(out.float().cpu().numpy(), P.apply_abs_rope3d(x), "apply_abs_rope3d")


# ------------------- NA block with q prepared inside the attention kernel
NA_BLOCK_CASES = [
    # (B, (T, H, W), NH, HD, kernel, norm, rope)  -> launched kernel family
    (1, (3, 8, 20), 4, 64, (3, 7, 7), True, True),        # pipe, 16-key segments, D=64
    (1, (3, 9, 37), 2, 128, (3, 7, 7), True, True),       # pipe, D=128, ragged x
    (1, (5, 13, 21), 2, 64, (5, 11, 11), True, True),     # deep bricks (stage-5 family), D=64, odd T
    (1, (4, 9, 24), 2, 64, (3, 11, 11), True, True),      # 32-wide tall bricks (t window 3), D=64
    (1, (2, 7, 30), 8, 128, (1, 3, 17), True, True),      # 32-key segments, head remap (NH % 8 == 0)
    (1, (2, 4, 40), 1, 128, (1, 3, 31), True, True),      # per-wave kernel (kw' > 25)
    (2, (2, 5, 9), 3, 64, (3, 3, 5), False, True),        # rope only
    (1, (2, 6, 10), 2, 128, (3, 5, 5), True, False),      # norm and scale only
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,grid,NH,HD,ks,norm,rope", NA_BLOCK_CASES)
def test_na3d_block_attention_fused_q(gpu, B, grid, NH, HD, ks, norm, rope):
    """The block's q preparation (per-head RMSNorm, * head_dim**-0.5 in bf16,
    absolute RoPE; diffusion_vae.py:263-277) done inside the NA kernel as it
    loads q: against the oracle (prologue oracle, then the NA oracle) at the
    attention bar, and bit for bit against the separate path (the one-pass
    prologue kernel, then the NA kernel), whose rounding points and
    per-head summation order the fused kernel reproduces."""
    from vidax_amd import (create_abs_rope3d_axis_freqs, create_abs_rope3d_freqs, na3d_block_attention,
                           na3d_qk_norm_rope, neighborhood_attention_3d)
    from vidax_amd import _lib
    print(f"[case] na3d fused q B={B} grid={grid} NH={NH} HD={HD} kernel={ks} norm={norm} rope={rope}", flush=True)
    rng = np.random.default_rng(sum(grid) * NH + HD + ks[2])
    shape = (B, *grid, NH, HD)
    q = _bf16_normal(rng, shape, 2.0)
    k_raw = _bf16_normal(rng, shape, 2.0)
    v = _bf16_normal(rng, shape)
    wq = (1.0 + 0.3 * rng.standard_normal(HD)).astype(np.float32) if norm else None
    wk = (1.0 + 0.3 * rng.standard_normal(HD)).astype(np.float32) if norm else None
    post = HD ** -0.5
    freqs = create_abs_rope3d_freqs(*grid, HD, device=gpu) if rope else None
    tq, tv = _dev(q, gpu), _dev(v, gpu)
    tw = torch.from_numpy(wq).to(gpu) if norm else None
    tk = na3d_qk_norm_rope(_dev(k_raw, gpu), torch.from_numpy(wk).to(gpu) if norm else None, freqs)
    fused = na3d_block_attention(tq, tk, tv, ks, tw, freqs)
    launched = _lib.last_launch()
    separate = neighborhood_attention_3d(na3d_qk_norm_rope(tq, tw, freqs, post_scale=post), tk, tv, ks)
    torch.cuda.synchronize()
    print(f"  launched {launched}", flush=True)
    assert launched == _lib.last_launch()
    assert torch.equal(fused, separate), "fused q preparation differs from the two-pass path"
    if rope:
        # the per-axis tables (t, h and w rows) give the same bits
        axes = create_abs_rope3d_axis_freqs(*grid, HD, device=gpu)
        fused_ax = na3d_block_attention(tq, tk, tv, ks, tw, axes)
        torch.cuda.synchronize()
        assert _lib.last_launch() == launched
        assert torch.equal(fused_ax, fused), "per-axis rope tables differ from the per-token tables"
    q_ref = P.na3d_qk_norm_rope(q, wq, post_scale=post, rope=rope)
    k_ref = tk.float().cpu().numpy()
    ref = A.na3d(q_ref, k_ref, v, ks)
    o = fused.float().cpu().numpy()
    d = np.abs(o - ref)
    print(f"  vs oracle: max_abs={d.max():.3e} mean_abs={d.mean():.3e}", flush=True)
    assert d.max() <= 2e-2 and d.mean() <= 2e-3
