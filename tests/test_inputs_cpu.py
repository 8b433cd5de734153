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


def _layer_records(names, t=0.0, dur=10.0):
    """Kernel records (start, end, name) of one flushed layer: the flush, then `names` back
    to back."""
    recs = [(t, t + 100.0, "void at::native::reduce_kernel<512, 1>(...)")]
    t += 100.0
    for n in names:
        recs.append((t, t + dur, n))
        t += dur + 1.0
    return recs, t


def test_bench_attributes_layer_kernels_to_steps():
    """bench.py's in-layer attribution of the library's kernels to steps, on the kernel names
    of each layer form: the fp32 B=128 layer (2a2 rotating q_rope in its epilogue), the
    16-bit layer (2a2 doing 2b and 2c; 3d on NT weight-streaming tiles) and the B=1 layer
    (q_small_kernel for 2b + 2c, out_small_kernel for 3d)."""
    import bench
    ns = "void mla::(anonymous namespace)::"
    args = "(mla::(anonymous namespace)::GemmArgs)"
    g = lambda t: f"{ns}gemm_kernel<{t}>{args}"
    w = lambda t: f"{ns}wgemm_kernel<{t}>(mla::(anonymous namespace)::WArgs)"
    fp32 = [g("float, float, 64, 64, 2, 2, false, 0, 0, false, false, false"),
            f"{ns}rmsnorm_kernel<0, 16>(...)",
            g("float, float, 64, 64, 2, 2, false, 0, 0, false, false, true"),
            g("float, float, 128, 64, 2, 2, false, 0, 0, false, true, false"),
            f"{ns}flash32x_kernel<4>(...)",
            g("float, float, 64, 64, 2, 2, true, 1, 0, false, false, false")]
    recs, t = _layer_records(fp32)
    more, _ = _layer_records(fp32, t)
    r = bench.attribute_steps(recs + more)
    assert r["layers"] == 2 and r["folded"] == {"2a2": ("2b",)}
    assert all(r[s] == 10.0 for s in ("2a1", "2a-n", "2a2", "2c", "3abc", "3d"))
    assert "2b" not in r

    bf16 = [w("unsigned short, 64, 4, 1, 0, false"), f"{ns}rmsnorm_kernel<1, 8>(...)",
            w("unsigned short, 128, 4, 1, 2, false"),
            f"{ns}flash16x_kernel<unsigned short, false, true>(...)",
            w("unsigned short, 64, 4, 1, 0, true")]
    r = bench.attribute_steps(_layer_records(bf16)[0])
    assert r["folded"] == {"2a2": ("2b", "2c")}
    assert [s for s in ("2a1", "2a-n", "2a2", "2b", "2c", "3abc", "3d") if s in r] == \
        ["2a1", "2a-n", "2a2", "3abc", "3d"]

    b1 = [g("float, float, 32, 128, 1, 4, false, 0, 0, false, false, false"),
          f"{ns}rmsnorm_kernel<0, 16>(...)",
          g("float, float, 32, 128, 1, 4, false, 0, 0, false, false, false"),
          f"{ns}q_small_kernel(...)", f"{ns}flash32w_kernel(...)",
          f"{ns}flash_merge_kernel(...)", f"{ns}out_small_kernel(...)"]
    r = bench.attribute_steps(_layer_records(b1)[0])
    assert r["folded"] == {"2c": ("2b",)}
    assert r["3abc"] == 20.0 and r["2c"] == 10.0 and r["3d"] == 10.0 and "2b" not in r
    assert r["kernels_sum"] == 70.0
