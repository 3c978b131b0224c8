"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture, and each fixture agrees with
an independent computation (torch's scaled_dot_product_attention in float64
for full attention, the pure-Python brute force for the NA windows), so a
later change to the oracle cannot drift silently.
GPU: the HIP path, called through the public entry points, meets the parity
bar (max-abs <= 2e-2, mean-abs <= 2e-3) against every fixture.
"""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import attention_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
FLASH = sorted(glob.glob(os.path.join(GOLDEN, "flash_*.npz")))
NA = sorted(glob.glob(os.path.join(GOLDEN, "na3d_*.npz")))

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _load(path):
    z = np.load(path)  # allow_pickle stays False
    d = {k: z[k] for k in z.files}
    for k in ("q", "k", "v"):
        d[k] = O.bits_to_f32(d[k])
    return d


def _name(p):
    return os.path.splitext(os.path.basename(p))[0]


def test_fixture_set_present():
    assert len(FLASH) >= 5 and len(NA) >= 3


@pytest.mark.parametrize("path", FLASH, ids=_name)
def test_oracle_reproduces_flash_fixture(path):
    d = _load(path)
    out = O.attention(d["q"], d["k"], d["v"], scale=float(d["scale"]), kv_len=d.get("kv_len"),
                      key_valid=d.get("key_valid"), key_bias=d.get("key_bias"))
    np.testing.assert_allclose(out, d["out"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("path", FLASH, ids=_name)
def test_flash_fixture_matches_torch_sdpa(path):
    """Independent library routine: SDPA in float64 with an additive mask."""
    d = _load(path)
    q, k, v = (torch.from_numpy(d[x]).double().permute(0, 2, 1, 3) for x in ("q", "k", "v"))
    B, H, Sq, _ = q.shape
    Sk = k.shape[2]
    add = torch.zeros(B, Sk, dtype=torch.float64)
    if "kv_len" in d:
        add[torch.arange(Sk)[None, :] >= torch.from_numpy(d["kv_len"]).long()[:, None]] = float("-inf")
    if "key_valid" in d:
        add[~torch.from_numpy(d["key_valid"]).bool()] = float("-inf")
    if "key_bias" in d:
        add = add + torch.from_numpy(d["key_bias"]).double()
    ref = torch.nn.functional.scaled_dot_product_attention(
        q, k, v, attn_mask=add[:, None, None, :].expand(B, H, Sq, Sk), scale=float(d["scale"]))
    np.testing.assert_allclose(ref.permute(0, 2, 1, 3).numpy(), d["out"], rtol=0, atol=1e-5)


@pytest.mark.parametrize("path", NA, ids=_name)
def test_oracle_reproduces_na_fixture(path):
    d = _load(path)
    out = O.na3d(d["q"], d["k"], d["v"], tuple(int(x) for x in d["kernel"]))
    np.testing.assert_allclose(out, d["out"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("path", NA, ids=_name)
def test_na_fixture_matches_brute_force(path):
    d = _load(path)
    ref = O.na3d_loops(d["q"], d["k"], d["v"], tuple(int(x) for x in d["kernel"]))
    np.testing.assert_allclose(ref, d["out"], rtol=0, atol=1e-5)


def _parity(o, ref, label):
    diff = np.abs(o.astype(np.float64) - ref.astype(np.float64))
    print(f"  {label}: max_abs={diff.max():.3e} mean_abs={diff.mean():.3e}", flush=True)
    assert np.isfinite(o).all(), label
    assert diff.max() <= MAX_ABS and diff.mean() <= MEAN_ABS, label


def _dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu).to(torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FLASH, ids=_name)
def test_hip_flash_matches_fixture(gpu, path):
    from vidax_amd import flash_attention
    print(f"[case] golden {_name(path)}", flush=True)
    d = _load(path)
    kw = {}
    for key in ("kv_len", "key_valid", "key_bias"):
        if key in d:
            kw[key] = torch.from_numpy(d[key]).to(gpu)
    out = flash_attention(_dev(d["q"], gpu), _dev(d["k"], gpu), _dev(d["v"], gpu),
                          scale=float(d["scale"]), **kw)
    torch.cuda.synchronize()
    _parity(out.float().cpu().numpy(), d["out"], _name(path))


@pytest.mark.gpu
@pytest.mark.parametrize("path", NA, ids=_name)
def test_hip_na3d_matches_fixture(gpu, path):
    from vidax_amd import neighborhood_attention_3d
    print(f"[case] golden {_name(path)}", flush=True)
    d = _load(path)
    out = neighborhood_attention_3d(_dev(d["q"], gpu), _dev(d["k"], gpu), _dev(d["v"], gpu),
                                    tuple(int(x) for x in d["kernel"]))
    torch.cuda.synchronize()
    _parity(out.float().cpu().numpy(), d["out"], _name(path))
