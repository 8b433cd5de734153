"""The layer replayed from a HIP graph (torch.cuda.CUDAGraph over the binding's calls).

The library launches only its own kernels on the caller's stream (no allocation, no
memset, no synchronisation), so a serving loop can capture a whole layer once and replay
it.  Each test captures q_absorbed + mla_attention (or the paged attention), replays the
graph several times with other eager work and synchronisations in between, and checks
every replay against the eager layer bit for bit (every kernel is deterministic), and the
eager layer against the float64 oracle on sampled inputs.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import mla_ref as R

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = R.DSV3


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


def _layer(ext, g, W_uk, W_uv):
    scale = math.sqrt(D.qk_head)

    def run():
        qa, qr = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"], W_uk,
                                g["positions"], D.nope, D.rope, 1e-6)
        return ext.mla_attention(qa, qr, g["c_kv"], g["pe_cache"], W_uv, scale)
    return run


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("B,Sk", [(2, 300), (3, 1000), (128, 300)])
def test_layer_graph_replay(ext, dtype, B, Sk):
    """Replays equal the eager layer bit for bit.  At B = 128 the 16-bit Q path runs the
    weight-streaming GEMMs with 2a2's fused epilogue and 2a-n's RoPE table."""
    inp = R.make_inputs(B, 1, Sk, seed=B + Sk)
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    g = {k: v.to(dtype).to(DEV) if v.is_floating_point() else v.to(DEV)
         for k, v in inp.items()}
    W_uk_d, W_uv_d = W_uk.to(dtype).to(DEV), W_uv.to(dtype).to(DEV)
    layer = _layer(ext, g, W_uk_d, W_uv_d)
    eager = layer()
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = layer()
    other = {k: (v * 0.5 if v.is_floating_point() else v) for k, v in g.items()}
    other_layer = _layer(ext, other, W_uk_d, W_uv_d)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager)
        other_layer()                   # eager work on other inputs between replays
        torch.cuda.synchronize()

    if dtype == torch.float32:
        ref = R.mla_layer(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], inp["wkv_b"],
                          inp["c_kv"], inp["pe_cache"], inp["positions"])
        torch.testing.assert_close(eager.cpu(), ref, rtol=1e-4, atol=1e-4)


def test_paged_attention_graph_replay(ext):
    """The paged attention (block table, ragged lengths) replays the same way.  The lengths
    are device data read by the replayed kernels, so a captured decode step stays valid as
    they change: between replays they grow by one key, then become equal (the dense split
    rule), then ragged again; every replay equals an eager call on the same lengths bit for
    bit."""
    B, page, lens = 3, 64, [700, 64, 1]
    mp = -(-max(lens) // page) + 1
    g = torch.Generator().manual_seed(21)
    qa = torch.randn(B, 1, D.n_heads, D.kv_rank, generator=g)
    qr = torch.randn(B, 1, D.n_heads, D.rope, generator=g)
    ck = torch.randn(B * mp, page, D.kv_rank, generator=g)
    pe = torch.randn(B * mp, page, D.rope, generator=g)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g)
    table = torch.randperm(B * mp, generator=g).to(torch.int32).reshape(B, mp)
    sl = torch.tensor(lens, dtype=torch.int32)
    args = [t.to(DEV) for t in (qa, qr, ck, pe, table, sl, wuv)]
    sl_dev = args[5]
    scale = math.sqrt(D.qk_head)
    eager = ext.mla_attention_paged(*args, scale)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = ext.mla_attention_paged(*args, scale)
    schedule = [lens, [n + 1 for n in lens], [300] * B, [5, 64 * mp, 100], lens]
    for step_lens in schedule:
        sl_dev.copy_(torch.tensor(step_lens, dtype=torch.int32))   # in place: same address
        torch.cuda.synchronize()
        eager = ext.mla_attention_paged(*args, scale).clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager), f"replay differs from eager at lengths {step_lens}"
        ext.mla_attention_paged(*args[:6], args[6] * 2.0, scale)   # other eager work
        torch.cuda.synchronize()
    ref = R.mla_attention_paged(qa, qr, ck, pe, table, torch.tensor(lens, dtype=torch.int32),
                                wuv, scale)
    torch.testing.assert_close(out_g.cpu(), ref, rtol=1e-4, atol=1e-4)
