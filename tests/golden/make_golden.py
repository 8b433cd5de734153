"""Write the small fp64 golden fixtures under tests/golden/.

The reference commits no golden vectors, and its Python oracle is never run here.  The
expected outputs in these fixtures therefore come from ``tests/brute_mla.py``, a
scalar-loop restatement of the layer's mathematics that shares no code with the oracle.
Inputs are seeded (numpy PCG64) and stored alongside, so the fixtures are self-contained.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import brute_mla  # noqa: E402

CASES = {
    # name: (B, Sq, Sk, hidden, H, q_lora, R, nope, rope, v, causal, seed)
    "tiny_noncausal": (2, 3, 5, 6, 2, 4, 4, 2, 4, 3, False, 11),
    "tiny_causal": (2, 3, 5, 6, 2, 4, 4, 2, 4, 3, True, 12),
    "small_noncausal": (2, 3, 37, 64, 4, 32, 32, 16, 16, 16, False, 13),
    "small_causal": (1, 4, 9, 32, 2, 16, 16, 8, 8, 8, True, 14),
}


def make_case(B, Sq, Sk, hidden, H, q_lora, R, nope, rope, v, causal, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, Sq, hidden))
    W_q_a = rng.standard_normal((hidden, q_lora)) / math.sqrt(hidden)
    gain = 1.0 + 0.1 * rng.standard_normal(q_lora)
    W_q_b = rng.standard_normal((q_lora, H * (nope + rope))) / math.sqrt(q_lora)
    wkv_b = rng.standard_normal((H, nope + v, R)) / math.sqrt(R)
    c_kv = rng.standard_normal((B, Sk, R))
    pe = rng.standard_normal((B, Sk, rope))
    positions = np.arange(Sk - Sq, Sk, dtype=np.int64)
    out = brute_mla.layer(x.tolist(), W_q_a.tolist(), gain.tolist(), W_q_b.tolist(),
                          wkv_b.tolist(), c_kv.tolist(), pe.tolist(), positions.tolist(),
                          H, nope, rope, v, causal=causal)
    return dict(x=x, W_q_a=W_q_a, q_norm_w=gain, W_q_b=W_q_b, wkv_b=wkv_b, c_kv=c_kv,
                pe_cache=pe, positions=positions, out=np.asarray(out),
                dims=np.array([B, Sq, Sk, hidden, H, q_lora, R, nope, rope, v, int(causal)]))


def main():
    for name, args in CASES.items():
        arrs = make_case(*args)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrs)
        print(f"wrote {path}  out shape {arrs['out'].shape}")


if __name__ == "__main__":
    main()
