"""GPU parity of streaming attention (bounded key chunks + online-softmax merge).

* vs the materialised path (mla_attention) on the same GPU tensors, with chunks small
  enough to force many merges, causal and not, fp32 and bf16;
* vs the CPU oracle on small shapes;
* the chunked-prefill configuration at full size (B=4, Sq=128, Sk=32768, causal): a causal
  query s sees exactly keys 0 .. Sk-Sq+s, so its oracle value is the non-causal oracle on
  the cache truncated there -- evaluated for a few (b, s) rows.
Tolerance fp32: rtol/atol 1e-4 (output); against the materialised path 1e-5 (the two
differ only by the order of the softmax rescaling).
"""

from __future__ import annotations

import math

import pytest
import torch

import attn_cases as C
from oracle import mla_ref as R

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = R.DSV3
SCALE = math.sqrt(D.qk_head)


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


def inputs(B, Sq, Sk, seed, dtype=torch.float32, layer_spread=False):
    """Queries ~ N(0,1) (the reference's check_3d inputs: scores with standard deviation
    sqrt(3)), or with the layer's spread (unit standard deviation, tests/attn_cases.py)."""
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(dtype).to(DEV)  # noqa: E731
    qs = (C.LAYER_QA_STD, C.LAYER_QR_STD) if layer_spread else (1.0, 1.0)
    return (mk(B, Sq, D.n_heads, D.kv_rank, sc=qs[0]), mk(B, Sq, D.n_heads, D.rope, sc=qs[1]),
            mk(B, Sk, D.kv_rank), mk(B, Sk, D.rope),
            mk(D.n_heads, D.v, D.kv_rank, sc=1 / math.sqrt(D.kv_rank)))


@pytest.mark.parametrize("B,Sq,Sk,causal,chunk", [(2, 1, 4989, False, 512), (1, 16, 1000, True, 128),
                                                  (3, 5, 700, True, 256), (1, 1, 16384, False, 0),
                                                  (2, 2, 300, False, 1024)])
def test_streaming_equals_materialised(ext, B, Sq, Sk, causal, chunk):
    args = inputs(B, Sq, Sk, seed=Sk + chunk)
    ref = ext.mla_attention(*args, SCALE, causal)
    got = ext.mla_attention_streaming(*args, SCALE, causal, chunk)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)


def test_streaming_bf16_equals_materialised(ext):
    args = inputs(2, 4, 2000, seed=7, dtype=torch.bfloat16, layer_spread=True)
    ref = ext.mla_attention(*args, SCALE, True)
    got = ext.mla_attention_streaming(*args, SCALE, True, 256)
    assert got.dtype == torch.bfloat16
    torch.testing.assert_close(got.float(), ref.float(), **C.tol(torch.bfloat16, ref.float()))
    oracle = R.mla_attention_official(*(t.cpu().float() for t in args), SCALE, causal=True)
    torch.testing.assert_close(got.float().cpu(), oracle, **C.tol(torch.bfloat16, oracle))


@pytest.mark.parametrize("causal", [False, True])
def test_streaming_vs_oracle(ext, causal):
    qa, qr, ck, pe, wuv = inputs(2, 8, 777, seed=11)
    got = ext.mla_attention_streaming(qa, qr, ck, pe, wuv, SCALE, causal, 128).cpu()
    ref = R.mla_attention_official(*(t.cpu().double() for t in (qa, qr, ck, pe, wuv)), SCALE,
                                   causal=causal).float()
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)


def test_chunked_prefill_long_context_full_size(ext):
    """B=4, Sq=128, Sk=32768, causal, fp32, DeepSeek-V3 dims, queries with the layer's
    spread (scores of unit standard deviation)."""
    B, Sq, Sk = 4, 128, 32768
    qa, qr, ck, pe, wuv = inputs(B, Sq, Sk, seed=5, layer_spread=True)
    out = ext.mla_attention_streaming(qa, qr, ck, pe, wuv, SCALE, True).cpu()
    assert out.shape == (B, Sq, D.n_heads, D.v) and torch.isfinite(out).all()
    for b, s in [(0, 0), (1, 63), (3, 127)]:
        lim = Sk - Sq + s + 1   # keys visible to query s
        ref = R.mla_attention_official(qa[b:b + 1, s:s + 1].cpu(), qr[b:b + 1, s:s + 1].cpu(),
                                       ck[b:b + 1, :lim].cpu(), pe[b:b + 1, :lim].cpu(),
                                       wuv.cpu(), SCALE)
        torch.testing.assert_close(out[b, s], ref[0, 0], rtol=1e-4, atol=1e-4)
