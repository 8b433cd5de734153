"""bench.py's synthetic inputs (mla-cuda_amd/mla_inputs.py) are bit-identical to the
oracle's seeded inputs, so a parity figure reported by bench.py refers to the same data the
GPU parity tests use."""

import torch

import mla_inputs
from oracle import mla_ref as R


def test_bench_inputs_equal_oracle_inputs():
    dims = mla_inputs.Dims(hidden=64, n_heads=4, q_lora=32, kv_rank=32, nope=16, rope=16, v=16)
    odims = R.MLADims(hidden=64, n_heads=4, q_lora=32, kv_rank=32, nope=16, rope=16, v=16)
    for dt in (torch.float32, torch.bfloat16):
        a = mla_inputs.make_inputs(3, 2, 37, dims, seed=5, dtype=dt)
        b = R.make_inputs(3, 2, 37, odims, seed=5, dtype=dt)
        assert a.keys() == b.keys()
        for k in a:
            assert a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]), k


def test_default_dims_are_deepseek_v3():
    d = mla_inputs.DEEPSEEK_V3
    assert (d.hidden, d.n_heads, d.q_lora, d.kv_rank, d.nope, d.rope, d.v) == \
        (R.DSV3.hidden, R.DSV3.n_heads, R.DSV3.q_lora, R.DSV3.kv_rank, R.DSV3.nope,
         R.DSV3.rope, R.DSV3.v)
