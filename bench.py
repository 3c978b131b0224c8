"""Benchmark of the flash-attention hot path on one MI355X.

Default workload: non-causal self-attention B=1, H=40, L=32760, D=128 in
bf16 (Wan2.1-14B 480p, 81 frames; latent grid 21x30x52), inputs ~ N(0,1)
resident in HBM. One "step" is one call of the kernel over that batch.
Prints ONE JSON line with the attention TFLOP/s, the fraction of MI355X dense
bf16 MFMA peak, ms per call, the roofline record of the kernel and a CPU
baseline timed on this host (the oracle's fp32 restatement on a bounded
sample of the same workload).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "attention TFLOP/s + % bf16 MFMA peak at L=32760 H=40 D=128; ms/call"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
# dense bf16 flop per shader clock cycle of the whole chip: 256 CUs x 4
# matrix cores x 1024 flop (2.517 PFLOP/s at 2.4 GHz, quoted as 2.5)
PEAK_BF16_FLOP_PER_CYCLE = 256 * 4 * 1024

WORKLOADS = {
    # name: (kind, params, description)
    "self_L32760_H40": ("flash", dict(B=1, Sq=32760, Sk=32760, H=40, seed=1),
                        "self-attention B=1 H=40 L=32760 D=128 (Wan2.1-14B 480p 81f)"),
    "self_L7800_H12": ("flash", dict(B=1, Sq=7800, Sk=7800, H=12, seed=0),
                       "self-attention B=1 H=12 L=7800 D=128 (Wan2.1-1.3B)"),
    "cross_L32760x512_B2": ("flash", dict(B=2, Sq=32760, Sk=512, H=40, seed=2, kv_len=(20, 512)),
                            "cross-attention B=2 H=40 Lq=32760 Lk=512, kv_len ~ U{20..512}"),
    "joint_L119056_H24": ("flash", dict(B=1, Sq=119056, Sk=119056, H=24, seed=4, tail_pad=(0, 200)),
                          "joint self-attention B=1 H=24 S=33*45*80+256, last 0-200 keys masked "
                          "(masked_self_attention)"),
    "self_key_bias_L32760_H40": ("flash", dict(B=1, Sq=32760, Sk=32760, H=40, seed=1, key_bias_pad=(100, 300)),
                                 "self-attention B=1 H=40 L=32760 D=128 with Cosmos3's (B,1,1,Sk) padding bias: "
                                 "0 on valid keys, -inf on a mid-sequence run of 100-300 keys "
                                 "(cosmos3/dit_layers.py:124-135), through dot_product_attention"),
    "self_rand_key_bias_L32760_H40": ("flash", dict(B=1, Sq=32760, Sk=32760, H=40, seed=1, key_bias_pad=(100, 300),
                                                    key_bias_randn=True),
                                      "self-attention B=1 H=40 L=32760 D=128 with a general (B,1,1,Sk) additive "
                                      "key bias: N(0,1) values, -inf on a mid-sequence run of 100-300 keys"),
    "t5_rel_bias_L512_H8_D64": ("flash", dict(B=2, Sq=512, Sk=512, H=8, D=64, seed=7, scale=1.0, t5_bias=True),
                                "UMT5 encoder attention B=2 L=512 H=8 D=64, scale 1, (1,H,L,L) relative-position "
                                "bias + (B,1,1,L) padding mask"),
    "na3d_21x45x80_H24": ("na3d", dict(B=1, T=21, Hs=45, W=80, NH=24, kernel=(3, 7, 7), seed=3),
                          "3D neighbourhood attention 21x45x80, window (3,7,7), B=1 NH=24 D=128"),
    "na3d_stage5_33x88x160_H4_D64": ("na3d", dict(B=1, T=33, Hs=88, W=160, NH=4, D=64, kernel=(11, 11, 11),
                                                  seed=6),
                                     "3D neighbourhood attention 33x88x160, window (11,11,11), B=1 NH=4 D=64 "
                                     "(LTX-2.5 VAE stage 5 head layout)"),
    "na3d_wide_x_21x45x80_H24": ("na3d", dict(B=1, T=21, Hs=45, W=80, NH=24, kernel=(3, 7, 31), seed=3),
                                 "3D neighbourhood attention 21x45x80, window (3,7,31) (x window above 25: the "
                                 "per-wave kernel), B=1 NH=24 D=128"),
    "na3d_block_fused_q_21x45x80_H24": ("na3d_block", dict(B=1, T=21, Hs=45, W=80, NH=24, kernel=(3, 7, 7), seed=3,
                                                          fused=True),
                                        "NA block attention 21x45x80 (3,7,7) NH=24 D=128: q RMSNorm + "
                                        "scale + abs RoPE inside the NA kernel"),
    "na3d_block_two_pass_21x45x80_H24": ("na3d_block", dict(B=1, T=21, Hs=45, W=80, NH=24, kernel=(3, 7, 7),
                                                            seed=3, fused=False),
                                         "NA block attention 21x45x80 (3,7,7) NH=24 D=128: q prologue pass, "
                                         "then the NA kernel"),
    "na3d_block_fused_q_stage5_33x88x160_H4_D64": ("na3d_block", dict(B=1, T=33, Hs=88, W=160, NH=4, D=64,
                                                                      kernel=(11, 11, 11), seed=6, fused=True),
                                                   "NA block attention 33x88x160 (11,11,11) NH=4 D=64: q prep "
                                                   "inside the NA kernel"),
    "na3d_block_two_pass_stage5_33x88x160_H4_D64": ("na3d_block", dict(B=1, T=33, Hs=88, W=160, NH=4, D=64,
                                                                       kernel=(11, 11, 11), seed=6, fused=False),
                                                    "NA block attention 33x88x160 (11,11,11) NH=4 D=64: q "
                                                    "prologue pass, then the NA kernel"),
    "qk_norm_rope_L32760_H40": ("prologue", dict(B=1, grid=(21, 30, 52), H=40, seed=5),
                                "q and k RMSNorm(5120) + 3D RoPE, B=1 L=32760 (21x30x52) H=40 D=128"),
}
DEFAULT_WORKLOAD = "self_L32760_H40"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def _flash_inputs(p, dev):
    import numpy as np
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(p["seed"])
    B, Sq, Sk, H, D = p["B"], p["Sq"], p["Sk"], p["H"], p.get("D", 128)
    q = torch.randn((B, Sq, H, D), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((B, Sk, H, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((B, Sk, H, D), generator=g, device=dev).to(torch.bfloat16)
    kw = {}
    valid_keys = [Sk] * B
    rng = np.random.default_rng(p["seed"])
    if "kv_len" in p:
        lo, hi = p["kv_len"]
        kvl = rng.integers(lo, hi + 1, size=B).astype(np.int32)
        kw["kv_len"] = torch.from_numpy(kvl).to(dev)
        valid_keys = [int(x) for x in kvl]
    if "tail_pad" in p:
        lo, hi = p["tail_pad"]
        pad = rng.integers(lo, hi + 1, size=B)
        valid = torch.ones((B, Sk), dtype=torch.bool, device=dev)
        for b in range(B):
            if pad[b]:
                valid[b, Sk - int(pad[b]):] = False
        kw["key_valid"] = valid
        from vidax_amd.attention import _last_valid_plus_one
        kw["kv_len"] = _last_valid_plus_one(valid)
        valid_keys = [Sk - int(x) for x in pad]
    if "key_bias_pad" in p:
        lo, hi = p["key_bias_pad"]
        n_pad = int(rng.integers(lo, hi + 1))
        if p.get("key_bias_randn"):
            bias = torch.randn((B, Sk), generator=g, device=dev)
        else:
            bias = torch.zeros((B, Sk), device=dev)
        s0 = Sk // 3
        bias[:, s0:s0 + n_pad] = float("-inf")
        kw["key_bias"] = bias
        valid_keys = [Sk - n_pad] * B
    if p.get("t5_bias"):
        # learned relative-position bias (1, H, L, L) plus a padding mask: the
        # second batch item's last 200 keys are padding
        bias = torch.randn((1, H, Sq, Sk), generator=g, device=dev)
        pad = torch.zeros((B, 1, 1, Sk), device=dev)
        pad[1, ..., Sk - 200:] = float("-inf")
        kw["bias"] = bias + pad
        kw["scale"] = p.get("scale", 1.0)
        valid_keys = [Sk, Sk - 200]
    return q, k, v, kw, valid_keys


def _flash_work(p, valid_keys):
    """Algorithmic flops and HBM bytes per call (q, o and the valid k, v once,
    plus a per-(query, key) bias once)."""
    H, D, Sq = p["H"], p.get("D", 128), p["Sq"]
    flops = 4.0 * H * D * Sq * sum(valid_keys)
    bytes_ = 2.0 * (p["B"] * Sq * H * D * 2) + 2.0 * sum(valid_keys) * H * D * 2
    if p.get("t5_bias"):
        bytes_ += 4.0 * H * Sq * p["Sk"]
    return flops, bytes_


def _na3d_work(p):
    B, T, Hs, W, NH, D = p["B"], p["T"], p["Hs"], p["W"], p["NH"], p.get("D", 128)
    kt, kh, kw = (min(p["kernel"][0], T), min(p["kernel"][1], Hs), min(p["kernel"][2], W))
    n = T * Hs * W
    flops = 4.0 * B * NH * n * kt * kh * kw * D
    bytes_ = 2.0 * 4 * B * n * NH * D
    return flops, bytes_


def _cpu_baseline(kind, p, budget_s=12.0):
    """Times the oracle's fp32 restatement on a bounded sample of the workload
    on this host's cores and scales it to the metric's unit (TFLOP/s)."""
    import numpy as np
    from oracle import attention_oracle as O
    try:
        from threadpoolctl import threadpool_info
        threads = max([d.get("num_threads", 1) for d in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    rng = np.random.default_rng(1234)
    if kind == "flash":
        H, Sk, D = 1, p["Sk"], p.get("D", 128)
        rows = 1024
        q = O.bf16_round(rng.standard_normal((1, rows, H, D), dtype=np.float32))
        k = O.bf16_round(rng.standard_normal((1, Sk, H, D), dtype=np.float32))
        v = O.bf16_round(rng.standard_normal((1, Sk, H, D), dtype=np.float32))
        O.attention(q[:, :64], k, v, acc=np.float32)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            O.attention(q, k, v, acc=np.float32, q_block=256)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 1000:
                break
        flops = 4.0 * D * rows * Sk * H * reps
        sample = (f"oracle fp32 (numpy/BLAS) attention, {reps} x (1 head x {rows} query rows x "
                  f"{Sk} keys, D={D}) of this workload, {el:.1f} s")
        return {"value": round(flops / el / 1e12, 6), "unit": "TFLOP/s", "cores": int(threads),
                "kind": "port", "sample": sample}
    if kind == "na3d_block":
        kind = "na3d"
    if kind == "prologue":
        from oracle import prologue_oracle as P
        S, L = 2048, p["H"] * 128
        x = O.bf16_round(rng.standard_normal((1, S, L), dtype=np.float32))
        w = np.ones(L, np.float32)
        cos, sin = P.create_rope3d_freqs(1, 32, 64, 128)
        reps, t0 = 0, time.perf_counter()
        while True:
            P.qk_norm_rope(x, w, cos, sin, p["H"])
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 1000:
                break
        gbs = 2.0 * 2 * S * L * reps / el / 1e9
        sample = f"oracle fp32 (numpy) RMSNorm+RoPE of {S} tokens x {L}, {reps} reps, {el:.1f} s"
        return {"value": round(gbs, 3), "unit": "GB/s", "cores": int(threads), "kind": "port", "sample": sample}
    # na3d: a slab of up to 3 planes of the H x W grid (24 rows of it for
    # windows wider than 8 x 8), two heads
    T, D = min(3, p["T"]), p.get("D", 128)
    Hs = p["Hs"] if p["kernel"][1] * p["kernel"][2] <= 64 else min(p["Hs"], 24)
    shape = (1, T, Hs, p["W"], 2, D)
    q = O.bf16_round(rng.standard_normal(shape, dtype=np.float32))
    k = O.bf16_round(rng.standard_normal(shape, dtype=np.float32))
    v = O.bf16_round(rng.standard_normal(shape, dtype=np.float32))
    reps, t0 = 0, time.perf_counter()
    while True:
        O.na3d(q, k, v, p["kernel"], acc=np.float32)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 200:
            break
    kt, kh, kw = (min(p["kernel"][0], T), min(p["kernel"][1], Hs), min(p["kernel"][2], p["W"]))
    flops = 4.0 * 2 * T * Hs * p["W"] * kt * kh * kw * D * reps
    sample = f"oracle fp32 NA3D on a (1,{T},{Hs},{p['W']},2,{D}) slab, {reps} reps, {el:.1f} s"
    return {"value": round(flops / el / 1e12, 6), "unit": "TFLOP/s", "cores": int(threads),
            "kind": "port", "sample": sample}


def _traffic(kernel_name, workload):
    """HBM bytes per launch of the kernel on this workload, measured with the
    FETCH_SIZE and WRITE_SIZE counters (two separate profiler passes) and
    scaled by the same counters' reading for a plain copy of known size."""
    try:
        with open(TRAFFIC_FILE) as f:
            stored = json.load(f)
    except (OSError, ValueError):
        return None
    rec = stored.get("workloads", {}).get(workload, {})
    # a figure measured on other kernel sources (any file under csrc/) is stale
    if rec.get("kernel") != kernel_name or stored.get("csrc_sha256_16") != _csrc_hash():
        return None
    return rec.get("hbm_bytes_per_launch")


def _csrc_hash():
    """First 16 hex digits of the SHA-256 of the kernel sources (vidax_amd/csrc,
    sorted by path), which the stored traffic figures were measured with."""
    import glob
    import hashlib
    csrc = os.path.join(ROOT, "vidax_amd", "csrc")
    paths = sorted(p for ext in ("*.hip", "*.hpp", "*.h", "*.cpp") for p in glob.glob(os.path.join(csrc, ext)))
    h = hashlib.sha256()
    for p in paths:
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


class _ClockStamps:
    """The shader clock the chip held over the timed loop. The clock moves
    with board power (a busy matrix core holds a lower clock, +-10 % between
    boxes and between launches), so a kernel's rate depends on it. A stamp
    (vx_debug_clock_stamp: 1024 one-wave workgroups, each storing its XCD,
    its hardware id, the shader clock counter and the real-time counter) is
    launched on the kernel's stream right before the loop and right after
    it. The shader counter is kept per CU, so the stamps are paired by CU
    (XCD, shader engine, CU): shader cycles passed / real time passed is that
    CU's clock over the loop. The XCDs hold different clocks (a spread of
    ~7 % at full load), so the mean over the CUs is reported: the figure
    GRBM_GUI_ACTIVE (summed over the 8 XCDs) / 8 / duration gives."""

    GROUPS = 1024

    def __init__(self, dev):
        import torch
        self.buf = torch.zeros((2, 4 * self.GROUPS), dtype=torch.int64, device=dev)
        self.khz = []

    def stamp(self, i, stream):
        import ctypes
        from vidax_amd import _lib
        khz = ctypes.c_int32(0)
        rc = _lib.lib().vx_debug_clock_stamp(self.buf[i].data_ptr(), self.GROUPS, ctypes.byref(khz),
                                             ctypes.c_void_p(stream.cuda_stream))
        _lib.raise_for(rc)
        self.khz.append(khz.value)

    def result(self):
        """{"mean", "median", "min", "max" (MHz over the CUs), "cus"} after a synchronize, or None."""
        if len(self.khz) != 2 or self.khz[0] <= 0:
            return None
        a = self.buf.cpu().numpy().reshape(2, self.GROUPS, 4)
        first = []
        for i in range(2):
            d = {}
            for xcc, hw, cyc, real in a[i]:
                d.setdefault((int(xcc), (int(hw) >> 8) & 0xFF), (int(cyc), int(real)))
            first.append(d)
        per = []
        for key in sorted(set(first[0]) & set(first[1])):
            (c0, r0), (c1, r1) = first[0][key], first[1][key]
            real = (r1 - r0) / (self.khz[0] * 1e3)
            if c1 > c0 and real > 0:
                per.append((c1 - c0) / real / 1e6)
        if not per:
            return None
        per.sort()
        return {"median": per[len(per) // 2], "mean": sum(per) / len(per), "min": per[0], "max": per[-1],
                "cus": len(per), "source": "s_memtime / s_memrealtime stamps around the timed loop, paired per CU"}


def _copy_calibration(mib, steps):
    """A plain device copy of known size, timed the same way; profiled with the
    same counters it gives the bytes-per-KiB factor of FETCH_SIZE/WRITE_SIZE."""
    import torch
    n = int(mib) << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": steps}), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 20; with the default warm-up, more for short calls: "
                         "enough for --timed-ms)")
    ap.add_argument("--timed-ms", type=float, default=100.0)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps before the timed ones (default: at least 3 and at least "
                         "--warmup-ms of GPU work, so the timed steps run at the clock the chip holds "
                         "under sustained load)")
    ap.add_argument("--warmup-ms", type=float, default=250.0)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB --steps times")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: the attention kernels run on a single GPU here; "
              "--gpus N with N > 1 is not supported (a sharded run would split "
              "heads or query tiles over the GPUs, one process each)", file=sys.stderr)
        return 2

    if args.copy_calibration_mib:
        return _copy_calibration(args.copy_calibration_mib, args.steps)

    import torch
    import vidax_amd
    from vidax_amd import _lib

    _lib.lib()
    dev = torch.device("cuda:0")
    kind, p, desc = WORKLOADS[args.workload]
    if kind == "flash":
        q, k, v, kw, valid_keys = _flash_inputs(p, dev)
        out = torch.empty_like(q)
        flops, bytes_ = _flash_work(p, valid_keys)

        if "tail_pad" in p:
            # HunyuanVideo's joint text+video attention, through its entry
            # point (hunyuan_video/common/dit_layers.py:264-337): a key
            # validity mask, valid keys a prefix
            def step():
                vidax_amd.masked_self_attention(q, k, v, key_valid=kw["key_valid"])
        elif "key_bias_pad" in p:
            # a (B, 1, 1, Sk) key bias through dot_product_attention
            # (src/vidax/core/attention.py:467-533), as Cosmos3 passes it
            kb4 = kw["key_bias"][:, None, None, :]

            def step():
                vidax_amd.dot_product_attention(q, k, v, bias=kb4)
        else:
            def step():
                vidax_amd.flash_attention(q, k, v, out=out, **kw)
    elif kind == "prologue":
        from vidax_amd.prologue import create_rope3d_freqs, qk_norm_rope
        g = torch.Generator(device=dev)
        g.manual_seed(p["seed"])
        S = p["grid"][0] * p["grid"][1] * p["grid"][2]
        L = p["H"] * 128
        qx = torch.randn((p["B"], S, L), generator=g, device=dev).to(torch.bfloat16)
        kx = torch.randn((p["B"], S, L), generator=g, device=dev).to(torch.bfloat16)
        wq = 1.0 + 0.1 * torch.randn(L, generator=g, device=dev)
        wk = 1.0 + 0.1 * torch.randn(L, generator=g, device=dev)
        freqs = create_rope3d_freqs(*p["grid"], 128, device=dev)
        flops = 0.0
        # read and write q and k once (bf16) plus the cos/sin tables once per tensor
        bytes_ = 2.0 * (2 * 2 * p["B"] * S * L) + 2.0 * (2 * S * 64 * 4)

        def step():
            qk_norm_rope(qx, wq, freqs, p["H"])
            qk_norm_rope(kx, wk, freqs, p["H"])
    elif kind == "na3d_block":
        from vidax_amd import create_abs_rope3d_axis_freqs, create_abs_rope3d_freqs, na3d_block_attention
        from vidax_amd import na3d_qk_norm_rope
        from vidax_amd import neighborhood_attention_3d
        g = torch.Generator(device=dev)
        g.manual_seed(p["seed"])
        D = p.get("D", 128)
        shape = (p["B"], p["T"], p["Hs"], p["W"], p["NH"], D)
        q = (2.0 * torch.randn(shape, generator=g, device=dev)).to(torch.bfloat16)
        k = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)  # k as the block prepares it
        v = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
        wq = 1.0 + 0.1 * torch.randn(D, generator=g, device=dev)
        out = torch.empty_like(q)
        flops, bytes_ = _na3d_work(p)
        if p["fused"]:
            # the fused kernel reads the per-axis rows (t, h and w tables)
            freqs = create_abs_rope3d_axis_freqs(p["T"], p["Hs"], p["W"], D, device=dev)

            def step():
                na3d_block_attention(q, k, v, p["kernel"], wq, freqs, out=out)
        else:
            freqs = create_abs_rope3d_freqs(p["T"], p["Hs"], p["W"], D, device=dev)

            def step():
                neighborhood_attention_3d(na3d_qk_norm_rope(q, wq, freqs, post_scale=D ** -0.5), k, v, p["kernel"])
    else:
        g = torch.Generator(device=dev)
        g.manual_seed(p["seed"])
        D = p.get("D", 128)
        shape = (p["B"], p["T"], p["Hs"], p["W"], p["NH"], D)
        q = (torch.randn(shape, generator=g, device=dev) * D ** -0.5).to(torch.bfloat16)
        k = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
        out = torch.empty_like(q)
        flops, bytes_ = _na3d_work(p)
        from vidax_amd.natten import na3d_attention

        def step():
            na3d_attention(q, k, v, p["kernel"], out=out)

    # Warm-up. Under sustained load the chip holds a power-limited shader
    # clock, but after any idle period of a few milliseconds it starts a burst
    # fast, drops below that clock for ~10 ms and recovers over ~20 ms more:
    # a 0.34 ms call ran 0.34 ms for 5 steps, 0.39-0.45 ms for the next 10
    # and 0.35 ms only after 40. So the untimed steps run back to back, in
    # chunks of ~20 ms with one synchronisation each, until --warmup-ms of
    # wall time has passed (unless --warmup is given), everything the timed
    # loop needs is made before them, and the timed loop covers at least
    # --timed-ms (unless --steps is given).
    stream = torch.cuda.current_stream(dev)
    clock = _ClockStamps(dev)
    if args.warmup is not None:
        n_warm = max(1, args.warmup)
        if args.steps is None:
            args.steps = 20
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        for _ in range(n_warm):
            step()
    else:
        step()  # (the first call also loads the kernels)
        torch.cuda.synchronize()
        t_w = time.perf_counter()
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        n_warm = 3
        est = max((time.perf_counter() - t_w) / 2, 1e-5)
        if args.steps is None:
            args.steps = max(20, int(args.timed_ms * 1e-3 / est) + 1)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        chunk = max(1, int(0.02 / est))
        while (time.perf_counter() - t_w) * 1e3 < args.warmup_ms:
            for _ in range(chunk):
                step()
            n_warm += chunk
            torch.cuda.synchronize()
    kernel_name = _lib.last_launch()  # the kernel the step launched (the last one, for two launches)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    clock.stamp(0, stream)
    ev[0].record(stream)
    for i in range(args.steps):
        step()
        ev[i + 1].record(stream)
    clock.stamp(1, stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    sclk = clock.result()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]
    ms = sum(per) / len(per)
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = bytes_ / (ms * 1e-3) / 1e9
    if kind == "prologue":
        tflops = 0.0
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                    "traffic": _traffic(kernel_name, args.workload)}
    elif kind == "flash":
        roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                    "traffic": _traffic(kernel_name, args.workload)}
    elif flops / bytes_ > PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9):
        # a wide window (e.g. 11^3) lies right of the ridge: matrix-core bound
        roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                    "traffic": _traffic(kernel_name, args.workload)}
    else:
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                    "traffic": _traffic(kernel_name, args.workload)}
    # The shader clock held over the timed loop, and the work per clock cycle
    # at that clock: flop/cycle over PEAK_BF16_FLOP_PER_CYCLE is the
    # matrix-core fraction independent of the clock the box held.
    roofline["sclk_mhz"] = round(sclk["mean"], 1) if sclk else None
    if sclk:
        roofline["sclk"] = {k: (round(v, 1) if isinstance(v, float) else v) for k, v in sclk.items()}
        cycles = ms * 1e-3 * sclk["mean"] * 1e6
        if flops:
            roofline["flop_per_cycle"] = round(flops / cycles, 1)
            roofline["frac_of_peak_at_sclk"] = round(flops / cycles / PEAK_BF16_FLOP_PER_CYCLE, 4)
        roofline["bytes_per_cycle"] = round(bytes_ / cycles, 1)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(kind, p, args.cpu_budget)
    value, unit = round(tflops, 2), "TFLOP/s"
    if kind == "prologue":
        value, unit = round(gbs, 1), "GB/s"
    rec = {
        "metric": METRIC,
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": n_warm,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 inputs resident in HBM",
        "config": {"workload": desc, "B": p["B"], "heads": p.get("H", p.get("NH")), "head_dim": p.get("D", 128),
                   "kernel": kernel_name},
        "pct_bf16_mfma_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "ms_per_call": round(ms, 4),
        "ms_per_call_min": round(min(per), 4),
        "algorithmic_gbs": round(gbs, 1),
        "wall_s": round(wall, 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
