"""Full-shape parity for the reference's published scenario matrix.

The reference's suite runs ten production shapes, all non-causal and fp32
(exhaustive_benchmark_suite.py:78-174), and gates each whole output against its PyTorch
formulation (:466-471).  Here every scenario runs at its full shape through the drop-in calls
(q_absorbed, then the fused mla_attention), and every output row is checked against the CPU
oracle at the north-star fp32 tolerance (rtol/atol 1e-4): the Q path whole against the oracle
from x, the attention against the oracle on the GPU's own q_absorbed / q_rope (so each stage is
held to its own accuracy), computed per sequence and per block of queries to bound host memory.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import mla_ref as R

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = R.DSV3
SCALE = math.sqrt(D.qk_head)
TOL = dict(rtol=1e-4, atol=1e-4)

SCENARIOS = [
    ("decode_single_user_long_ctx", 1, 1, 65536),
    ("decode_serving_avg_ctx", 128, 1, 4989),
    ("decode_serving_long_ctx", 128, 1, 8192),
    ("decode_serving_high_batch", 256, 1, 2048),
    ("decode_speculative_2tok", 64, 2, 512),
    ("decode_speculative_4tok", 64, 4, 768),
    ("decode_speculative_long_ctx", 132, 4, 4096),
    ("prefill_chat_batch", 8, 512, 512),
    ("prefill_chunk_2k", 1, 2048, 2048),
    ("prefill_chunk_4k", 1, 4096, 4096),
]


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


@pytest.mark.parametrize("name,B,Sq,Sk", SCENARIOS, ids=[s[0] for s in SCENARIOS])
def test_reference_scenario_full_shape(ext, name, B, Sq, Sk):
    print(f"scenario {name}: B={B} Sq={Sq} Sk={Sk}", flush=True)
    inp = R.make_inputs(B, Sq, Sk, seed=3)
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    g = {k: v.to(DEV) for k, v in inp.items()}
    qa, qr = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"],
                            W_uk.contiguous().to(DEV), g["positions"], D.nope, D.rope, 1e-6)
    out = ext.mla_attention(qa, qr, g["c_kv"], g["pe_cache"], W_uv.contiguous().to(DEV), SCALE)
    qa, qr, out = qa.cpu(), qr.cpu(), out.cpu()
    del g
    assert out.shape == (B, Sq, D.n_heads, D.v) and torch.isfinite(out).all()

    rqa, rqr = R.prepare_q_mla_absorbed(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                        W_uk, inp["positions"], D.nope, D.rope)
    torch.testing.assert_close(qa, rqa, **TOL)
    torch.testing.assert_close(qr, rqr, **TOL)

    # the attention for every (sequence, query) row, in blocks of queries
    qblk = max(1, 256 // max(1, Sk // 4096))
    for b in range(B):
        for s0 in range(0, Sq, qblk):
            s1 = min(Sq, s0 + qblk)
            ref = R.mla_attention_official(qa[b:b + 1, s0:s1], qr[b:b + 1, s0:s1],
                                           inp["c_kv"][b:b + 1], inp["pe_cache"][b:b + 1],
                                           W_uv, SCALE)
            torch.testing.assert_close(out[b:b + 1, s0:s1], ref, **TOL,
                                       msg=lambda m: f"sequence {b}, queries {s0}:{s1}: {m}")
