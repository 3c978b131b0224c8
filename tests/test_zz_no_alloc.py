"""GPU test of vx_flash_attn_noalloc_fwd, the allocation-free entry point:
its key-split partials live in the library's static device scratch. Two
calls in a row (the second on a smaller problem, so stale scratch contents
from the first are present) must match vx_flash_attn_ws_fwd, the entry point
with a caller-provided workspace, bit for bit, and the oracle within the bar."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import attention_oracle as O

pytestmark = pytest.mark.gpu


def _call(entry, q, k, v, out, kv_len=None, ws=None):
    from vidax_amd import _lib
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            kv_len.data_ptr() if kv_len is not None else None, None, None, 0, B, Sq, Sk, H, D,
            None, None, None, None, ctypes.c_float(D ** -0.5)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    L = _lib.lib()
    if entry == "noalloc":
        rc = L.vx_flash_attn_noalloc_fwd(*args, stream)
    else:
        rc = L.vx_flash_attn_ws_fwd(*args, ws.data_ptr() if ws is not None else None,
                                    ws.numel() if ws is not None else 0, stream)
    _lib.raise_for(rc)
    return _lib.last_launch()


def test_noalloc_matches_workspace_entry(gpu):
    from vidax_amd import _lib
    cases = [
        # B, Sq, Sk, H, seed, kv_len: the first splits 220 of 732 items (28 MiB of
        # scratch), the second every one of its 24 items over a smaller span
        (1, 7800, 7800, 12, 180, None),
        (2, 700, 2100, 2, 181, [700, 2100]),
    ]
    for B, Sq, Sk, H, seed, kvl in cases:
        print(f"[case] noalloc B={B} Sq={Sq} Sk={Sk} H={H} kv_len={kvl}", flush=True)
        q, k, v, _ = O.make_flash_inputs(B, Sq, Sk, H, 128, seed)
        t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu).to(torch.bfloat16)
        tq, tk, tv = t(q), t(k), t(v)
        kv_len = torch.tensor(kvl, dtype=torch.int32, device=gpu) if kvl is not None else None
        ws_bytes = int(_lib.lib().vx_flash_attn_workspace_size(B, Sq, Sk, H, 128))
        assert ws_bytes > 0
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
        out_na = torch.empty_like(tq)
        out_ws = torch.empty_like(tq)
        name_na = _call("noalloc", tq, tk, tv, out_na, kv_len)
        name_ws = _call("ws", tq, tk, tv, out_ws, kv_len, ws)
        torch.cuda.synchronize()
        print(f"  launched {name_na} / {name_ws}", flush=True)
        assert name_na == name_ws == "flash_fwd_split_kernel<0, 128, 4>"
        assert torch.equal(out_na, out_ws), "noalloc output differs from the workspace entry point"
        rows = np.unique(np.linspace(0, Sq - 1, 64).astype(int))
        ref = O.attention(q[:, rows], k, v, kv_len=np.array(kvl, np.int32) if kvl is not None else None)
        err = np.abs(out_na[:, torch.from_numpy(rows).to(gpu)].float().cpu().numpy() - ref)
        print(f"  vs oracle: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3


def test_noalloc_under_graph_capture(gpu):
    """The use the entry point exists for: captured into a HIP graph (torch's
    CUDAGraph, global capture mode, in which a device allocation inside the
    capture fails) after one eager warm-up call, then replayed. Between
    replays the program runs its own eager work, including an eager call on
    a smaller problem that overwrites the shared scratch; every replay must
    equal the eager result bit for bit."""
    B, Sq, Sk, H, seed = 1, 7800, 7800, 12, 182   # splits 220 of 732 items into the scratch
    print(f"[case] noalloc graph capture B={B} Sq={Sq} Sk={Sk} H={H}", flush=True)
    q, k, v, _ = O.make_flash_inputs(B, Sq, Sk, H, 128, seed)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu).to(torch.bfloat16)
    tq, tk, tv = t(q), t(k), t(v)
    out_eager = torch.empty_like(tq)
    assert _call("noalloc", tq, tk, tv, out_eager) == "flash_fwd_split_kernel<0, 128, 4>"  # warm-up
    torch.cuda.synchronize()
    # a smaller problem whose split also goes through the scratch
    q2, k2, v2, _ = O.make_flash_inputs(2, 700, 2100, 2, 128, seed + 1)
    sq2, sk2, sv2 = t(q2), t(k2), t(v2)
    out2 = torch.empty_like(sq2)

    out_g = torch.empty_like(tq)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _call("noalloc", tq, tk, tv, out_g)
    for r in range(4):
        out_g.fill_(7.0)                               # eager work between replays
        _call("noalloc", sq2, sk2, sv2, out2)          # dirties the scratch
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        same = torch.equal(out_g, out_eager)
        print(f"  replay {r}: equal to eager = {same}", flush=True)
        assert same, f"replay {r} differs from the eager call"
