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


def test_bench_torch_formulation_matches_oracle():
    """bench.py's same-GPU library baseline (torch_layer) computes the oracle's layer: run
    on the CPU at small dims, causal and not, it agrees with R.mla_layer."""
    import math
    import bench
    dims = mla_inputs.Dims(hidden=64, n_heads=4, q_lora=32, kv_rank=32, nope=16, rope=16, v=16)
    odims = R.MLADims(hidden=64, n_heads=4, q_lora=32, kv_rank=32, nope=16, rope=16, v=16)
    for causal in (False, True):
        g = mla_inputs.make_inputs(3, 5, 37, dims, seed=2)
        W_uk = g["wkv_b"][:, :dims.nope].contiguous()
        W_uv = g["wkv_b"][:, dims.nope:].contiguous()
        scale = math.sqrt(dims.qk_head)
        got = bench.torch_layer(g, W_uk, W_uv, dims, scale, causal=causal)
        ref = R.mla_layer(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"], g["wkv_b"], g["c_kv"],
                          g["pe_cache"], g["positions"], odims, causal=causal)
        torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)


def test_device_generated_inputs_have_the_same_shapes():
    dims = mla_inputs.Dims(hidden=64, n_heads=4, q_lora=32, kv_rank=32, nope=16, rope=16, v=16)
    a = mla_inputs.make_inputs(2, 3, 20, dims, seed=1)
    b = mla_inputs.make_inputs(2, 3, 20, dims, seed=1, device=torch.device("cpu"))
    for k in a:
        assert a[k].shape == b[k].shape and a[k].dtype == b[k].dtype, k
    assert torch.equal(a["positions"], b["positions"])


def test_bench_scenarios_are_the_reference_matrix():
    """The ten published scenarios (exhaustive_benchmark_suite.py:78-174) with their shapes,
    plus the two prefill shapes the reference leaves out for memory."""
    import bench
    published = {k: v[:3] for k, v in bench.SCENARIOS.items() if v[4] is not None}
    assert published == {
        "decode_single_user_long_ctx": (1, 1, 65536), "decode_serving_avg_ctx": (128, 1, 4989),
        "decode_serving_long_ctx": (128, 1, 8192), "decode_serving_high_batch": (256, 1, 2048),
        "decode_speculative_2tok": (64, 2, 512), "decode_speculative_4tok": (64, 4, 768),
        "decode_speculative_long_ctx": (132, 4, 4096), "prefill_chat_batch": (8, 512, 512),
        "prefill_chunk_2k": (1, 2048, 2048), "prefill_chunk_4k": (1, 4096, 4096)}
    assert len(bench.SCENARIOS) == 12
