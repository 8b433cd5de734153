"""GPU parity of the float64 path (MLA_DTYPE_F64).

The reference dispatches double through both launches (mla_kernels.cu:674, 1561) and its
dtype check holds the double output to 1e-13 of the float64 reference's largest element,
with the output dtype kept (check_dtypes.py:23-38, rows Sk=64 "plain" and Sk=16384
"split-K", B = Sq = 1, randn inputs).  The same bar here: the error of the HIP path's
double output relative to the largest element of the oracle (oracle/mla_ref.py in float64
on the CPU) is below 1e-13, on check_dtypes' own rows, on causal and batched shapes, on the
Q path (q_absorbed and q_rope, positions up to 4988) and on whole layers.
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
F64 = torch.float64
REL = 1e-13     # check_dtypes.py:23 (float64 row)


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


def rel_err(out, ref):
    return ((out.double() - ref).abs().max() / ref.abs().max()).item()


def gpu(t):
    return t.to(DEV)


@pytest.mark.parametrize("Sk", [64, 16384], ids=["plain", "split-K"])
def test_attention_f64_like_check_dtypes(ext, Sk):
    """check_dtypes.py's float64 rows: B = Sq = 1, randn inputs generated in float32 and
    cast to double, the output in double within 1e-13 of the float64 reference's max."""
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(F64)  # noqa: E731
    qa, qr = mk(1, 1, D.n_heads, D.kv_rank), mk(1, 1, D.n_heads, D.rope)
    ck, pe = mk(1, Sk, D.kv_rank), mk(1, Sk, D.rope)
    wuv = mk(D.n_heads, D.v, D.kv_rank)
    out = ext.mla_attention(*(gpu(t) for t in (qa, qr, ck, pe, wuv)), SCALE).cpu()
    assert out.dtype == F64
    ref = R.mla_attention_official(qa, qr, ck, pe, wuv, SCALE)
    assert rel_err(out, ref) < REL


@pytest.mark.parametrize("B,Sq,Sk,H,causal", [(2, 3, 300, 128, True), (3, 1, 1000, 128, False),
                                              (1, 8, 700, 128, True), (2, 5, 257, 40, False),
                                              (1, 1, 1, 128, False), (4, 2, 65, 7, True)])
def test_attention_f64_vs_oracle(ext, B, Sq, Sk, H, causal):
    """Batches, several queries, causal masks (key j visible to query i iff
    j <= Sk - Sq + i), row and key counts off the 64-wide tiles, a single key."""
    g = torch.Generator().manual_seed(B * 1000 + Sk)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=F64)  # noqa: E731
    qa, qr = mk(B, Sq, H, D.kv_rank) * 0.5, mk(B, Sq, H, D.rope)
    ck, pe = mk(B, Sk, D.kv_rank), mk(B, Sk, D.rope)
    wuv = mk(H, D.v, D.kv_rank) / math.sqrt(D.kv_rank)
    out = ext.mla_attention(*(gpu(t) for t in (qa, qr, ck, pe, wuv)), SCALE, causal).cpu()
    assert out.dtype == F64 and out.shape == (B, Sq, H, D.v)
    ref = R.mla_attention_official(qa, qr, ck, pe, wuv, SCALE, causal=causal)
    assert rel_err(out, ref) < REL


def run_q(ext, inp, positions=None):
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    pos = inp["positions"] if positions is None else positions
    return ext.q_absorbed(gpu(inp["x"]), gpu(inp["W_q_a"]), gpu(inp["q_norm_w"]),
                          gpu(inp["W_q_b"]), gpu(W_uk.contiguous()), gpu(pos), D.nope, D.rope,
                          1e-6)


@pytest.mark.parametrize("B,Sq", [(2, 3), (1, 1), (5, 2)])
def test_q_absorbed_f64_vs_oracle(ext, B, Sq):
    """The Q path in double (2a1, RMSNorm, 2a2, RoPE at positions Sk-Sq .. Sk-1 = 4988 at
    most, 2c) against the oracle's float64 formulation; the RoPE table is the float64 one
    the oracle evaluates (rope_inv_freq in float64)."""
    inp = R.make_inputs(B, Sq, 4989, seed=B + Sq, dtype=F64)
    qa, qr = run_q(ext, inp)
    assert qa.dtype == F64 and qr.dtype == F64
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    rqa, rqr = R.prepare_q_mla_absorbed(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                        W_uk, inp["positions"], D.nope, D.rope)
    assert rel_err(qa.cpu(), rqa) < REL
    assert rel_err(qr.cpu(), rqr) < REL


def test_q_absorbed_f64_per_sequence_positions(ext):
    inp = R.make_inputs(3, 2, 8, seed=4, dtype=F64)
    pos = torch.tensor([[10, 11], [4987, 4988], [0, 1]])
    qa, qr = run_q(ext, inp, pos)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    rqa, rqr = R.prepare_q_ragged(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], W_uk,
                                  pos, D.nope, D.rope)
    assert rel_err(qa.cpu(), rqa) < REL
    assert rel_err(qr.cpu(), rqr) < REL


@pytest.mark.parametrize("B,Sq,Sk,causal", [(1, 1, 512, False), (8, 1, 4989, False),
                                            (2, 16, 1000, True)])
def test_layer_f64_vs_oracle(ext, B, Sq, Sk, causal):
    """Whole layers in double: cfg1's shape, the B=8 decode of the small-batch sweep, and a
    causal chunk, every sequence against the oracle's float64 layer."""
    inp = R.make_inputs(B, Sq, Sk, seed=7, dtype=F64)
    qa, qr = run_q(ext, inp)
    _, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    out = ext.mla_attention(qa, qr, gpu(inp["c_kv"]), gpu(inp["pe_cache"]),
                            gpu(W_uv.contiguous()), SCALE, causal).cpu()
    assert out.dtype == F64
    ref = R.mla_layer(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], inp["wkv_b"],
                      inp["c_kv"], inp["pe_cache"], inp["positions"], causal=causal)
    assert rel_err(out, ref) < REL


def test_f64_mixed_dtypes_and_per_step_ops_refuse(ext):
    """Mixed float64 / float32 operands are refused, and so are the per-step ops, which
    keep float32 intermediates: float64 is for the two fused calls."""
    qa = torch.randn(1, 1, D.n_heads, D.kv_rank, dtype=F64, device=DEV)
    qr = torch.randn(1, 1, D.n_heads, D.rope, dtype=F64, device=DEV)
    ck = torch.randn(1, 8, D.kv_rank, dtype=F64, device=DEV)
    pe = torch.randn(1, 8, D.rope, dtype=F64, device=DEV)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, dtype=F64, device=DEV)
    with pytest.raises(RuntimeError, match="dtype"):
        ext.mla_attention(qa, qr, ck.float(), pe, wuv, SCALE)
    with pytest.raises(RuntimeError, match="float64"):
        ext.gemm(qa.reshape(D.n_heads, D.kv_rank), wuv[0].t().contiguous())
