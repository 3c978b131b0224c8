"""CPU tests that pin the oracle before it is trusted as the GPU checker.

The reference ships no golden vectors for this path (and its JAX code cannot
be imported here), so the oracle is pinned by: an independent library routine
(torch's scaled_dot_product_attention on the CPU), hand-derived known answers
(NATTEN window tables), closed forms and invariants, and a brute-force loop
version of the neighbourhood attention. Each check is chosen so that a
plausible mistake fails it; `test_planted_mistakes_are_caught` plants such
mistakes in a copy of the oracle's arithmetic and shows the checks fire.
"""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as O


def _sdpa(q, k, v, scale, valid=None, bias=None, attn_mask=None):
    """torch SDPA in float64 on (B, S, H, D) numpy inputs."""
    tq = torch.from_numpy(np.asarray(q, np.float64)).permute(0, 2, 1, 3)
    tk = torch.from_numpy(np.asarray(k, np.float64)).permute(0, 2, 1, 3)
    tv = torch.from_numpy(np.asarray(v, np.float64)).permute(0, 2, 1, 3)
    mask = None
    if valid is not None:
        mask = torch.from_numpy(valid)[:, None, None, :]
    if bias is not None:
        mask = torch.from_numpy(np.asarray(bias, np.float64))[:, None, None, :]
    if attn_mask is not None:
        mask = attn_mask
    out = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=scale)
    return out.permute(0, 2, 1, 3).numpy()


# ----------------------------------------------------------------- bf16
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10,
        np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0, -0.0, 65504.0, 1e-40,
                  3.3895314e38, np.inf, -np.inf], dtype=np.float32),
    ])
    ours = O.bf16_to_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    # ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert O.bf16_round(np.array([1.0 + 2 ** -8], np.float32))[0] == 1.0


# ------------------------------------------------------- NATTEN windows
@pytest.mark.parametrize("L,K,expected", [
    (5, 3, [0, 0, 1, 2, 2]),
    (4, 3, [0, 0, 1, 1]),
    (2, 3, [0, 0]),                 # K clamped to L = 2
    (7, 7, [0] * 7),
    (10, 4, [0, 0, 0, 1, 2, 3, 4, 5, 6, 6]),  # even K: start = i - 2
    (9, 7, [0, 0, 0, 0, 1, 2, 2, 2, 2]),
    (1, 5, [0]),
])
def test_window_start_known_answers(L, K, expected):
    np.testing.assert_array_equal(O.window_start(L, K), expected)


@pytest.mark.parametrize("L", [1, 2, 3, 8, 21, 45, 80])
@pytest.mark.parametrize("K", [1, 2, 3, 5, 7, 11])
def test_window_invariants(L, K):
    idx = O.window_indices(L, K)
    kk = min(K, L)
    assert idx.shape == (L, kk)
    assert idx.min() >= 0 and idx.max() <= L - 1
    for i in range(L):
        assert idx[i, 0] <= i <= idx[i, -1]          # a query sees itself
    s = O.window_start(L, K)
    assert np.all(np.diff(s) >= 0) and np.all(np.diff(s) <= 1)  # slides by at most one


# ------------------------------------------------------- full attention
@pytest.mark.parametrize("B,Sq,Sk,H,D", [(1, 5, 7, 2, 16), (2, 33, 64, 3, 128), (1, 1, 1, 1, 8)])
def test_attention_matches_torch_sdpa(B, Sq, Sk, H, D):
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((B, S, H, D)) for S in (Sq, Sk, Sk))
    for scale in (D ** -0.5, 1.0, 0.37):
        np.testing.assert_allclose(O.attention(q, k, v, scale=scale), _sdpa(q, k, v, scale),
                                   rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(O.attention(q, k, v), _sdpa(q, k, v, D ** -0.5), rtol=1e-10, atol=1e-12)


def test_attention_masks_match_torch_sdpa():
    rng = np.random.default_rng(2)
    B, Sq, Sk, H, D = 3, 17, 29, 2, 32
    q, k, v = (rng.standard_normal((B, S, H, D)) for S in (Sq, Sk, Sk))
    valid = rng.random((B, Sk)) > 0.4
    valid[:, 0] = True
    np.testing.assert_allclose(O.attention(q, k, v, key_valid=valid), _sdpa(q, k, v, D ** -0.5, valid=valid),
                               rtol=1e-10, atol=1e-12)
    bias = rng.standard_normal((B, Sk))
    bias[~valid] = -np.inf
    np.testing.assert_allclose(O.attention(q, k, v, key_bias=bias), _sdpa(q, k, v, D ** -0.5, bias=bias),
                               rtol=1e-10, atol=1e-12)
    kv_len = np.array([1, 15, 29])
    prefix = np.arange(Sk)[None, :] < kv_len[:, None]
    np.testing.assert_allclose(O.attention(q, k, v, kv_len=kv_len), _sdpa(q, k, v, D ** -0.5, valid=prefix),
                               rtol=1e-10, atol=1e-12)


def test_attention_full_bias_matches_torch_sdpa():
    """Head- and query-dependent additive bias (T5-style) and a causal boolean
    mask against torch's SDPA with the same (B, H, Sq, Sk) mask."""
    rng = np.random.default_rng(21)
    B, Sq, Sk, H, D = 2, 9, 9, 3, 16
    q, k, v = (rng.standard_normal((B, S, H, D)) for S in (Sq, Sk, Sk))
    bias = rng.standard_normal((1, H, Sq, Sk)) * 2
    causal = np.tril(np.ones((Sq, Sk), bool))
    full = bias + np.where(causal, 0.0, -np.inf)[None, None]
    ref = _sdpa(q, k, v, 1.0, attn_mask=torch.from_numpy(np.broadcast_to(full, (B, H, Sq, Sk)).copy()))
    np.testing.assert_allclose(O.attention(q, k, v, scale=1.0, bias=full), ref, atol=1e-10)


def test_attention_invariants():
    rng = np.random.default_rng(3)
    B, Sq, Sk, H, D = 2, 9, 13, 2, 16
    q, k, v = (rng.standard_normal((B, S, H, D)) for S in (Sq, Sk, Sk))
    kv_len = np.array([5, 13])
    # (i) Sk = 1 -> out = v
    np.testing.assert_allclose(O.attention(q, k[:, :1], v[:, :1]), np.broadcast_to(v[:, :1], q.shape), atol=1e-14)
    # (ii) q = 0 -> mean of the valid v rows (pins the mask exactly)
    out0 = O.attention(np.zeros_like(q), k, v, kv_len=kv_len)
    for b in range(B):
        np.testing.assert_allclose(out0[b], np.broadcast_to(v[b, :kv_len[b]].mean(0), out0[b].shape), atol=1e-13)
    # (iii) permuting keys together with their mask leaves the output unchanged
    perm = rng.permutation(Sk)
    valid = rng.random((B, Sk)) > 0.3
    valid[:, 0] = True
    np.testing.assert_allclose(O.attention(q, k[:, perm], v[:, perm], key_valid=valid[:, perm]),
                               O.attention(q, k, v, key_valid=valid), atol=1e-13)
    # (iv) one-hot q/k with a large scale gathers the matching v row
    qq = np.zeros((1, 4, 1, 8))
    kk = np.zeros((1, 6, 1, 8))
    for i in range(4):
        qq[0, i, 0, i + 1] = 1.0
    for j in range(6):
        kk[0, j, 0, j] = 1.0
    vv = rng.standard_normal((1, 6, 1, 8))
    np.testing.assert_allclose(O.attention(qq, kk, vv, scale=200.0)[0, :, 0], vv[0, 1:5, 0], atol=1e-12)
    # (v) a constant added to every logit of a row (a uniform key bias) changes nothing
    np.testing.assert_allclose(O.attention(q, k, v, key_bias=np.full((B, Sk), 3.25)), O.attention(q, k, v),
                               atol=1e-13)
    # (vi) ragged length == zero-padded keys excluded by the mask (the
    # reference's pad + segment-id construction, attention.py:264-278)
    pad = 128 - Sk
    kp = np.concatenate([k, np.zeros((B, pad, H, D))], axis=1)
    vp = np.concatenate([v, np.zeros((B, pad, H, D))], axis=1)
    np.testing.assert_allclose(O.attention(q, kp, vp, kv_len=np.array([Sk, Sk])), O.attention(q, k, v), atol=1e-13)
    # (vii) prefix kv_len == the same set as a boolean mask == as a -inf bias
    prefix = np.arange(Sk)[None, :] < kv_len[:, None]
    ref = O.attention(q, k, v, kv_len=kv_len)
    np.testing.assert_allclose(O.attention(q, k, v, key_valid=prefix), ref, atol=1e-14)
    np.testing.assert_allclose(O.attention(q, k, v, key_bias=np.where(prefix, 0.0, -np.inf)), ref, atol=1e-14)
    # (viii) key-only semantics: a padded *query* row still averages the valid keys
    qz = q.copy()
    qz[:, -1] = 0.0
    o = O.attention(qz, k, v, kv_len=kv_len)
    np.testing.assert_allclose(o[1, -1], v[1, :13].mean(0), atol=1e-13)
    # fully masked rows are zero (defined behaviour)
    assert np.all(O.attention(q, k, v, kv_len=np.array([0, 0])) == 0)


def test_attention_rows_is_exact_subset():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((2, S, 3, 16)) for S in (40, 50, 50))
    rows = np.array([0, 7, 39])
    np.testing.assert_allclose(O.attention_rows(q, k, v, rows, kv_len=np.array([9, 50])),
                               O.attention(q, k, v, kv_len=np.array([9, 50]))[:, rows], atol=1e-14)


def test_weight_rounding_mode_is_close():
    """The Hunyuan dense path rounds weights to bf16 (dit_layers.py:336); the
    effect stays far below the parity bar."""
    rng = np.random.default_rng(5)
    q, k, v = (O.bf16_round(rng.standard_normal((1, S, 2, 128)).astype(np.float32)) for S in (64, 300, 300))
    a = O.attention(q, k, v)
    b = O.attention(q, k, v, weights_dtype_round=True)
    assert np.abs(a - b).max() < 2e-3


# --------------------------------------------------- neighbourhood attention
@pytest.mark.parametrize("shape,ks", [
    ((1, 3, 4, 5, 2, 8), (3, 3, 3)),
    ((1, 2, 5, 6, 1, 8), (3, 5, 2)),   # kt clamped to T = 2, even kw
    ((2, 4, 3, 3, 1, 4), (1, 7, 7)),   # kh, kw clamped
    ((1, 5, 2, 7, 1, 4), (4, 1, 6)),
])
def test_na3d_matches_brute_force(shape, ks):
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal(shape) for _ in range(3))
    np.testing.assert_allclose(O.na3d(q, k, v, ks, scale=0.7), O.na3d_loops(q, k, v, ks, scale=0.7),
                               rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("shape,ks", [
    ((1, 3, 4, 5, 2, 8), (3, 3, 3)),
    ((1, 2, 5, 6, 1, 8), (3, 5, 2)),   # kt clamped to T = 2, even kw
    ((2, 4, 3, 3, 1, 4), (1, 7, 7)),   # kh, kw clamped
    ((1, 5, 2, 7, 1, 4), (4, 1, 6)),
    ((1, 4, 9, 11, 3, 8), (3, 7, 7)),  # the (3, 7, 7) window with borders on every side
])
def test_na3d_dense_matches_gather_and_brute_force(shape, ks):
    """The dense per-row form (two matrix products over each query row's key
    box, out-of-window box keys masked) used for whole-grid GPU checks
    equals the window-gather form and the brute force."""
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal(shape) for _ in range(3))
    dense = O.na3d_dense(q, k, v, ks, scale=0.7)
    np.testing.assert_allclose(dense, O.na3d(q, k, v, ks, scale=0.7), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dense, O.na3d_loops(q, k, v, ks, scale=0.7), rtol=1e-10, atol=1e-12)
    rows = [(0, 0), (shape[1] - 1, shape[2] - 1)]
    part = O.na3d_dense(q, k, v, ks, scale=0.7, ty_rows=rows)
    sel = tuple(np.array(rows).T)
    np.testing.assert_allclose(part[:, sel[0], sel[1]], dense[:, sel[0], sel[1]], rtol=1e-12, atol=1e-14)


def test_na3d_window_one_is_identity():
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 3, 4, 5, 2, 8)) for _ in range(3))
    np.testing.assert_allclose(O.na3d(q, k, v, (1, 1, 1)), v, atol=1e-14)


def test_na3d_full_window_is_full_attention():
    """A window covering the whole grid on every axis is plain attention over
    all T*H*W tokens (checked through torch SDPA, independent of both)."""
    rng = np.random.default_rng(8)
    B, T, Hs, W, NH, D = 1, 3, 4, 5, 2, 8
    q, k, v = (rng.standard_normal((B, T, Hs, W, NH, D)) for _ in range(3))
    out = O.na3d(q, k, v, (7, 9, 11), scale=0.5)
    flat = lambda x: x.reshape(B, T * Hs * W, NH, D)
    ref = _sdpa(flat(q), flat(k), flat(v), 0.5).reshape(out.shape)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_na3d_interior_translation():
    """Away from the borders, shifting the whole grid shifts the output."""
    rng = np.random.default_rng(9)
    shape = (1, 7, 9, 9, 1, 4)
    q, k, v = (rng.standard_normal(shape) for _ in range(3))
    ks = (3, 3, 3)
    out = O.na3d(q, k, v, ks)
    sh = lambda x: np.roll(x, shift=(1, 1, 1), axis=(1, 2, 3))
    out_s = O.na3d(sh(q), sh(k), sh(v), ks)
    # interior queries whose windows do not touch the border or the wrap
    np.testing.assert_allclose(out_s[:, 3:6, 3:8, 3:8], out[:, 2:5, 2:7, 2:7], atol=1e-12)


def test_na3d_dtype_points_are_within_bar():
    """The reference rounds logits and weights to bf16 (diffusion_vae.py:222-223);
    that changes the output well inside the 2e-2 / 2e-3 parity bar."""
    q, k, v = O.make_na3d_inputs(1, 3, 8, 10, 2, 128, seed=10)
    a = O.na3d(q, k, v, (3, 7, 7))
    b = O.na3d(q, k, v, (3, 7, 7), round_logits_bf16=True, round_weights_bf16=True)
    d = np.abs(a - b)
    assert d.max() < 1e-2 and d.mean() < 1e-3


# ------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught():
    """Plausible mistakes planted in copies of the oracle's arithmetic fail
    the independent checks used above."""
    rng = np.random.default_rng(11)
    B, Sq, Sk, H, D = 2, 6, 11, 2, 16
    q, k, v = (rng.standard_normal((B, S, H, D)) for S in (Sq, Sk, Sk))
    ref = _sdpa(q, k, v, D ** -0.5)

    def wrong_scale():
        return O.attention(q, k, v, scale=(D ** -0.5) ** 2)

    def off_by_one_mask():
        return O.attention(q, k, v, kv_len=np.array([Sk - 1, Sk]))

    def swapped_kv():
        return O.attention(q, v, k)

    def mixed_heads():
        return O.attention(q, k[:, :, ::-1], v)

    for bad in (wrong_scale, off_by_one_mask, swapped_kv, mixed_heads):
        assert not np.allclose(bad(), ref, atol=1e-6), bad.__name__

    # NA: a window start without the border clamp reads the wrong keys
    def bad_start(length, kernel):
        kk = min(kernel, length)
        return np.clip(np.arange(length) - kk // 2, 0, length - 1)
    good = O.window_start(9, 7)
    assert not np.array_equal(bad_start(9, 7), good)
