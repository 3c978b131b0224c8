"""Writes the golden fixtures in this directory from the CPU oracle (float64).

The reference ships no golden vectors for its attention path and cannot be
imported here, so these fixtures are the oracle's own outputs on small seeded
inputs. They pin the oracle against regressions (tests/test_golden.py checks
it reproduces them exactly) and give the GPU tests fixed expected outputs.

Inputs are stored as bf16 bit patterns (uint16), outputs as float32.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention_oracle as O  # noqa: E402

FLASH_CASES = {
    # name: (B, Sq, Sk, H, seed, mask, scale)
    "flash_small_unmasked": (1, 40, 70, 2, 100, None, None),
    "flash_ragged_kvlen": (2, 33, 130, 2, 101, ("kv_len", 1, 130), None),
    "flash_tail_pad": (2, 20, 77, 1, 102, ("tail_pad", 0, 30), None),
    "flash_scale_one": (1, 17, 65, 1, 103, None, 1.0),
    # Cosmos3-style additive key bias: -inf on a mid-sequence run, finite elsewhere
    "flash_key_bias": (2, 24, 96, 2, 104, "bias", None),
}
NA_CASES = {
    # name: ((B, T, H, W, NH), kernel, seed)
    "na3d_3x7x7": ((1, 3, 6, 10, 1), (3, 7, 7), 200),
    "na3d_clamped": ((1, 2, 3, 5, 2), (3, 5, 9), 201),
    "na3d_even": ((1, 4, 5, 6, 1), (2, 4, 2), 202),
}


def _bits(x):
    return O.bf16_to_bits(np.asarray(x, np.float32))


def main():
    for name, (B, Sq, Sk, H, seed, mask, scale) in FLASH_CASES.items():
        q, k, v, extra = O.make_flash_inputs(B, Sq, Sk, H, 128, seed, None if mask == "bias" else mask)
        if mask == "bias":
            rng = np.random.default_rng(seed + 1000)
            bias = (0.5 * rng.standard_normal((B, Sk))).astype(np.float32)
            bias[0, 10:30] = -np.inf
            bias[1, 50:51] = -np.inf
            bias[1, 80:] = -np.inf
            extra["key_bias"] = bias
        out = O.attention(q, k, v, scale=scale, kv_len=extra.get("kv_len"),
                          key_valid=extra.get("key_valid"), key_bias=extra.get("key_bias"))
        arrays = dict(q=_bits(q), k=_bits(k), v=_bits(v), out=out.astype(np.float32),
                      scale=np.float64(scale if scale is not None else 128 ** -0.5))
        if "kv_len" in extra:
            arrays["kv_len"] = extra["kv_len"]
        for key in ("key_valid", "key_bias"):
            if key in extra:
                arrays[key] = extra[key]
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    for name, ((B, T, Hs, W, NH), ks, seed) in NA_CASES.items():
        q, k, v = O.make_na3d_inputs(B, T, Hs, W, NH, 128, seed)
        out = O.na3d(q, k, v, ks)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), q=_bits(q), k=_bits(k), v=_bits(v),
                            out=out.astype(np.float32), kernel=np.array(ks, np.int32))
    print("wrote", len(FLASH_CASES) + len(NA_CASES), "fixtures to", HERE)


if __name__ == "__main__":
    main()
