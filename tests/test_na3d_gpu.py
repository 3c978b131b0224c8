"""GPU parity tests of the 3D neighbourhood-attention kernel against the oracle.

Same bar as the flash kernel: max-abs <= 2e-2, mean-abs <= 2e-3, plus a
mean-abs / RMS bound. q is pre-scaled (the reference's caller convention) and
the kernel is called with scale 1.0 through `neighborhood_attention_3d`.
"""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3
MEAN_REL_RMS = 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev).to(torch.bfloat16)


def _check(o, ref, label):
    d = np.abs(o.astype(np.float64) - ref)
    rms = float(np.sqrt(np.mean(ref ** 2))) + 1e-30
    mx, mean = float(d.max()), float(d.mean())
    print(f"  {label}: max_abs={mx:.3e} mean_abs={mean:.3e} mean/rms={mean / rms:.3e}", flush=True)
    assert np.isfinite(o).all(), f"{label}: non-finite output"
    assert mx <= MAX_ABS and mean <= MEAN_ABS and mean / rms <= MEAN_REL_RMS, label


NA_CASES = [
    # (B, T, H, W, NH), kernel, seed
    ((1, 3, 8, 16, 2), (3, 7, 7), 30),     # exact bricks
    ((1, 4, 6, 9, 2), (3, 5, 5), 31),      # ragged bricks (H % 4, W % 8)
    ((2, 2, 5, 7, 1), (3, 3, 3), 32),      # kt clamped to T
    ((1, 5, 13, 21, 3), (3, 7, 7), 33),
    ((1, 3, 9, 11, 1), (2, 4, 6), 34),     # even windows
    ((1, 2, 3, 4, 2), (5, 9, 9), 35),      # every window clamped: full attention
    ((1, 3, 4, 30, 1), (1, 1, 25), 36),    # wide x window (two 16-key segments)
    ((1, 2, 4, 70, 1), (1, 3, 57), 37),    # per-wave kernel, x box of 64 slots
    ((1, 3, 10, 40, 2), (3, 11, 11), 41),  # 32-slot x windows (LTX-2.5 stage-5 shape family)
    ((1, 4, 17, 33, 1), (3, 5, 13), 42),
    ((2, 5, 9, 65, 2), (5, 3, 9), 43),     # ragged workgroup bricks along y and x
    ((1, 2, 20, 8, 1), (2, 9, 3), 44),
    ((1, 3, 19, 37, 2), (3, 11, 11), 45),  # tall bricks (kw' 10-13), ragged along y (19 % 8) and x (37 % 16)
    ((2, 4, 9, 23, 1), (3, 13, 10), 46),   # tall bricks, widest x window (13) clamped in y
    ((1, 3, 5, 40, 2), (3, 3, 7), 47),     # x bricks 32-63: waves 1-3 hold no query (x >= 40)
    ((2, 2, 7, 20, 1), (2, 3, 9), 48),     # one x brick, wave 3 (x 24-31) empty; kw' = 9
]


def _expected_kernel(H, W, kw, D, T=1, kt=1):
    """The NA kernel for a clamped x window kw' = min(kw, W) (and t window
    kt' = min(kt, T)), written out here independently of the library's plan."""
    k = min(kw, W)
    if k <= 9:
        # head dim 64: 1 x 8 x 16 bricks unless they cover more of the y-x
        # plane than the 1 x 4 x 32 ones
        if D == 64 and -(-H // 8) * 8 * (-(-W // 16) * 16) <= -(-H // 4) * 4 * (-(-W // 32) * 32):
            return "na3d_tall_kernel<64>"
        # head dim 128 with a t window of 2 or more: bricks two t planes deep
        if D == 128 and min(kt, T) >= 2:
            return "na3d_tstack_kernel<128>"
        return f"na3d_pipe_kernel<16, {D}>"
    if k <= 13:
        # head dim 64: 32-wide bricks unless they leave more ragged columns
        if D == 64 and -(-W // 32) * 32 == -(-W // 16) * 16:
            # deep t windows: the 32-wide bricks two t planes deep
            return "na3d_deep_kernel<64>" if min(kt, T) >= 5 else "na3d_tall_wide_kernel<64>"
        return f"na3d_tall_kernel<{D}>"
    if k <= 25:
        return f"na3d_pipe_kernel<32, {D}>"
    return f"na3d_wave_kernel<{D}>"


def _run(gpu, shape, ks, seed, D):
    from vidax_amd import _lib, neighborhood_attention_3d
    B, T, H, W, NH = shape
    q, k, v = O.make_na3d_inputs(B, T, H, W, NH, D, seed)
    out = neighborhood_attention_3d(_t(q, gpu), _t(k, gpu), _t(v, gpu), ks)
    launched = _lib.last_launch()
    assert launched == _expected_kernel(H, W, ks[2], D, T, ks[0]), launched
    torch.cuda.synchronize()
    _check(out.float().cpu().numpy(), O.na3d(q, k, v, ks), f"oracle ({launched})")


@pytest.mark.parametrize("shape,ks,seed", NA_CASES)
def test_na3d_small(gpu, shape, ks, seed):
    _say(f"na3d shape={shape} kernel={ks} seed={seed}")
    _run(gpu, shape, ks, seed, 128)


NA_D64_CASES = [
    # LTX-2.5 diffusion-VAE head dim 64 (src/vidax/models/ltx2_5/configs.py:194-203)
    ((1, 3, 8, 16, 2), (3, 7, 7), 50),
    ((1, 4, 6, 9, 3), (3, 5, 5), 51),
    ((2, 5, 13, 21, 1), (3, 5, 5), 52),
    ((1, 12, 13, 24, 2), (11, 11, 11), 53),   # stage-5 window
    ((1, 3, 9, 40, 4), (3, 3, 25), 54),       # widest x window for head dim 64
    ((1, 13, 21, 35, 2), (11, 11, 11), 55),   # stage-5 window, ragged tall bricks
    ((1, 3, 12, 40, 2), (3, 9, 9), 56),       # empty waves at the ragged x edge
    ((1, 5, 19, 64, 2), (5, 11, 11), 57),     # 32-wide tall bricks, two along x, ragged y
    ((2, 4, 10, 56, 1), (3, 13, 12), 58),     # 32-wide tall bricks, even window, two empty waves at x
    ((1, 5, 11, 20, 2), (3, 7, 7), 59),       # stage-1 grid: 16-key segments (tall bricks would pad 11 rows to 16)
    ((1, 3, 4, 64, 1), (3, 3, 5), 65),        # 16-key segments, one y brick
    ((1, 4, 22, 40, 2), (3, 7, 7), 66),       # tall bricks at kw' = 7, ragged x (40 % 16)
    ((2, 3, 13, 21, 1), (3, 5, 9), 67),       # tall bricks at kw' = 9, ragged y and x, even area
    ((1, 7, 10, 32, 2), (7, 9, 11), 68),      # deep bricks: odd T (a last brick one plane deep), ragged y
    ((2, 6, 9, 30, 1), (5, 5, 13), 69),       # deep bricks at kt' = 5, ragged y and x, two batch items
    ((1, 5, 8, 32, 8), (5, 11, 11), 70),      # deep bricks, t window = T, y window clamped, eight heads
    ((2, 9, 6, 64, 1), (7, 13, 13), 71),      # deep bricks, widest tall x window, y window clamped to 6
]


@pytest.mark.parametrize("shape,ks,seed", NA_D64_CASES)
def test_na3d_head_dim_64(gpu, shape, ks, seed):
    _say(f"na3d D=64 shape={shape} kernel={ks} seed={seed}")
    _run(gpu, shape, ks, seed, 64)


# With num_heads % 8 == 0 the kernels remap workgroups so that all bricks of
# a head land on one XCD; these cases run that remap on every pipelined
# kernel (16- and 32-key segments, tall bricks) with ragged y and x edges.
NA_NH8_CASES = [
    # (B, T, H, W, NH), kernel, seed, D
    ((1, 3, 11, 21, 8), (3, 11, 11), 60, 64),    # tall, stage-5 window family, D=64
    ((1, 3, 11, 21, 8), (3, 11, 11), 61, 128),   # tall, D=128
    ((1, 2, 7, 37, 8), (3, 5, 17), 62, 128),     # 32-key segments (kw' = 17)
    ((1, 2, 6, 45, 8), (1, 3, 25), 63, 64),      # 32-key segments, widest D=64 window
    ((2, 3, 9, 19, 16), (3, 7, 7), 64, 128),     # 16-key segments, two batch items
]


@pytest.mark.parametrize("shape,ks,seed,D", NA_NH8_CASES)
def test_na3d_head_remap(gpu, shape, ks, seed, D):
    _say(f"na3d NH%8==0 shape={shape} kernel={ks} seed={seed} D={D}")
    _run(gpu, shape, ks, seed, D)


# Windows wider than 25 (any size, both head dims) run on the per-wave kernel,
# whose x box is round_up(kw' + 7, 16) slots: beyond 64 slots, ragged y/x
# bricks, the widest windows clamped to the grid.
NA_WIDE_CASES = [
    # (B, T, H, W, NH), kernel, seed, D
    ((1, 2, 5, 90, 1), (1, 3, 75), 70, 128),     # 96-slot x box
    ((1, 3, 6, 40, 2), (3, 3, 29), 71, 64),      # head dim 64 above 25
    ((1, 2, 5, 100, 1), (1, 5, 85), 72, 64),     # head dim 64, 96-slot x box
    ((2, 2, 9, 130, 1), (2, 3, 121), 73, 128),   # 128-slot x box, ragged y bricks, two batch items
    ((1, 2, 4, 64, 8), (2, 3, 60), 74, 64),      # NH = 8
]


@pytest.mark.parametrize("shape,ks,seed,D", NA_WIDE_CASES)
def test_na3d_wide_windows(gpu, shape, ks, seed, D):
    _say(f"na3d wide window shape={shape} kernel={ks} seed={seed} D={D}")
    _run(gpu, shape, ks, seed, D)


@pytest.mark.parametrize("shift", [-1000.0, -120.0, 200.0, 1000.0])
@pytest.mark.parametrize("D,H,W", [(128, 9, 20), (64, 9, 20), (64, 16, 16)])
def test_na3d_row_offsets(gpu, shift, D, H, W):
    """A constant added to every score of a query leaves its softmax
    unchanged: key dim 0 all ones, the query's dim 0 = `shift` on every other
    x position (0 elsewhere), so queries far below 2^-100 or far above 2^8
    (log2 units) sit next to ordinary ones in the same wave. The 16 x 16
    grid runs the tall bricks at head dim 64."""
    from vidax_amd import _lib, neighborhood_attention_3d
    _say(f"na3d row offsets shift={shift} D={D} grid 3x{H}x{W}")
    B, T, NH = 1, 3, 2
    rng = np.random.default_rng(71)
    q = O.bf16_round((0.3 * rng.standard_normal((B, T, H, W, NH, D))).astype(np.float32))
    k = O.bf16_round((0.3 * rng.standard_normal((B, T, H, W, NH, D))).astype(np.float32))
    v = O.bf16_round(rng.standard_normal((B, T, H, W, NH, D)).astype(np.float32))
    k[..., 0] = 1.0
    q[:, :, :, ::2, :, 0] = shift
    q[:, :, :, 1::2, :, 0] = 0.0
    out = neighborhood_attention_3d(_t(q, gpu), _t(k, gpu), _t(v, gpu), (3, 7, 7))
    assert _lib.last_launch() == _expected_kernel(H, W, 7, D, T, 3), _lib.last_launch()
    torch.cuda.synchronize()
    _check(out.float().cpu().numpy(), O.na3d(q, k, v, (3, 7, 7)), "oracle")


def test_na3d_window_one_is_identity(gpu):
    from vidax_amd import neighborhood_attention_3d
    _say("na3d window (1,1,1) identity")
    q, k, v = O.make_na3d_inputs(1, 3, 7, 10, 2, 128, 38)
    out = neighborhood_attention_3d(_t(q, gpu), _t(k, gpu), _t(v, gpu), (1, 1, 1))
    np.testing.assert_array_equal(out.float().cpu().numpy(), v)


def test_na3d_full_window_equals_flash(gpu):
    """A window covering the grid is full attention over the T*H*W tokens:
    the NA kernel must agree with the flash kernel on the flattened tokens."""
    from vidax_amd import flash_attention, neighborhood_attention_3d
    _say("na3d full window vs flash")
    B, T, H, W, NH = 1, 2, 4, 6, 2
    q, k, v = O.make_na3d_inputs(B, T, H, W, NH, 128, 39)
    tq, tk, tv = _t(q, gpu), _t(k, gpu), _t(v, gpu)
    out = neighborhood_attention_3d(tq, tk, tv, (T, H, W))
    flat = lambda x: x.reshape(B, T * H * W, NH, 128)
    ref = flash_attention(flat(tq), flat(tk), flat(tv), scale=1.0).reshape(out.shape)
    d = (out.float() - ref.float()).abs()
    assert d.max().item() <= 1e-2 and d.mean().item() <= 1e-3


def test_na3d_deterministic(gpu):
    from vidax_amd import neighborhood_attention_3d
    _say("na3d determinism")
    q, k, v = O.make_na3d_inputs(1, 3, 9, 17, 2, 128, 40)
    tq, tk, tv = _t(q, gpu), _t(k, gpu), _t(v, gpu)
    a = neighborhood_attention_3d(tq, tk, tv, (3, 7, 7))
    b = neighborhood_attention_3d(tq, tk, tv, (3, 7, 7))
    assert torch.equal(a, b)


@pytest.mark.slow
def test_na3d_config4_whole_grid(gpu):
    """Config shape: grid 21x45x80, window (3,7,7), B=1 NH=24 D=128: every
    query of the grid against the oracle (its dense per-row form, fp32 on
    BLAS), and 14 (t, y) rows against the reference's own dtype points."""
    from vidax_amd import neighborhood_attention_3d
    _say("na3d c4 21x45x80 NH=24 (3,7,7) whole grid")
    B, T, H, W, NH = 1, 21, 45, 80, 24
    q, k, v = O.make_na3d_inputs(B, T, H, W, NH, 128, 3)
    out = neighborhood_attention_3d(_t(q, gpu), _t(k, gpu), _t(v, gpu), (3, 7, 7))
    from vidax_amd import _lib
    assert _lib.last_launch() == "na3d_tstack_kernel<128>", _lib.last_launch()
    o = out.float().cpu().numpy()
    ref = O.na3d_dense(q, k, v, (3, 7, 7), acc=np.float32)
    _check(o, ref, "c4 whole grid")
    # the reference's own dtype points (bf16 logits and weights) stay within the bar too
    rows = [(0, 0), (0, 44), (20, 0), (20, 44), (1, 1), (10, 22), (10, 3), (19, 43),
            (5, 40), (15, 2), (2, 21), (18, 30), (11, 44), (9, 0)]
    ref_bf = O.na3d(q, k, v, (3, 7, 7), ty_rows=rows[:4], round_logits_bf16=True, round_weights_bf16=True)
    sel4 = tuple(np.array(rows[:4]).T)
    _check(o[0][sel4], ref_bf[0][sel4], "c4 rows vs bf16-logit reference")


@pytest.mark.slow
def test_na3d_stage5_sampled_rows(gpu):
    """LTX-2.5 VAE stage-5 shape at full size: grid 33x88x160, window
    (11,11,11), B=1 NH=4 D=64 (the 2 x 4 x 32 deep bricks); every query of
    64 sampled (t, y) rows against the oracle: 8 rows for each y mod 8 (each
    row's position in a brick of 4 y rows, twice), both t parities (the two
    planes of a brick), the t and y borders included; a row holds every x
    brick of the grid."""
    from vidax_amd import _lib, neighborhood_attention_3d
    _say("na3d stage 5 33x88x160 NH=4 D=64 (11,11,11) sampled rows")
    B, T, H, W, NH = 1, 33, 88, 160, 4
    q, k, v = O.make_na3d_inputs(B, T, H, W, NH, 64, 5)
    out = neighborhood_attention_3d(_t(q, gpu), _t(k, gpu), _t(v, gpu), (11, 11, 11))
    assert _lib.last_launch() == _expected_kernel(H, W, 11, 64, T, 11), _lib.last_launch()
    o = out.float().cpu().numpy()
    rng = np.random.default_rng(55)
    rows = {(0, 0), (32, 87), (16, 7), (16, 8), (5, 44), (27, 80), (1, 86), (31, 3)}
    for r in range(8):
        ys = [y for y in range(H) if y % 8 == r]
        ts = [0, T - 1] + [int(x) for x in rng.choice(np.arange(1, T - 1), size=6, replace=False)]
        yy = [ys[0], ys[-1]] + [int(x) for x in rng.choice(ys[1:-1], size=6, replace=False)]
        rows.update(zip(ts, yy))
    rows = sorted(rows)
    assert len(rows) >= 64 and len({y % 8 for _, y in rows}) == 8 and len({t % 2 for t, _ in rows}) == 2
    ref = O.na3d_dense(q, k, v, (11, 11, 11), acc=np.float32, ty_rows=rows)
    sel = tuple(np.array(rows).T)
    _check(o[0][sel], ref[0][sel], f"stage-5 {len(rows)} rows")


@pytest.mark.slow
def test_na3d_wide_window_sampled_rows(gpu):
    """The per-wave kernel at the c4 grid with a (3,7,31) window, B=1 NH=24
    D=128: every query of 6 sampled (t, y) rows against the oracle."""
    from vidax_amd import _lib, neighborhood_attention_3d
    _say("na3d 21x45x80 NH=24 (3,7,31) sampled rows")
    B, T, H, W, NH = 1, 21, 45, 80, 24
    q, k, v = O.make_na3d_inputs(B, T, H, W, NH, 128, 6)
    out = neighborhood_attention_3d(_t(q, gpu), _t(k, gpu), _t(v, gpu), (3, 7, 31))
    assert _lib.last_launch() == _expected_kernel(H, W, 31, 128, T, 3), _lib.last_launch()
    o = out.float().cpu().numpy()
    rows = [(0, 0), (20, 44), (10, 3), (10, 4), (7, 41), (13, 22)]
    ref = O.na3d(q, k, v, (3, 7, 31), ty_rows=rows)
    sel = tuple(np.array(rows).T)
    _check(o[0][sel], ref[0][sel], "wide-window rows")
