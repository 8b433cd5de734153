"""GPU parity of the path's neighbours: weight prep (wkv_b split), the KV-cache append and
the output projection wo, against the CPU oracle (``oracle/mla_ref.py``: ``split_wkv_b``,
``kv_append``, ``o_proj``; pinned in ``tests/test_oracle.py`` by brute force).

Tolerances: the wkv_b split is a copy and must be bit-exact; fp32 results rtol/atol 1e-4
(O(1) values after a 7168- or 16384-deep fp32 reduction); bf16 results rtol/atol 2e-2
against the fp32 oracle on the same bf16-rounded inputs.
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
TOL_BF16 = dict(rtol=2e-2, atol=2e-2)


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU (torch.cuda.is_available() is False)")
    import mla_custom_cuda  # noqa: F401  (fails loudly if the extension is not built)
    return mla_custom_cuda


def gpu(t):
    return t.to(DEV)


def kv_inputs(B, Sq, rows, seed, dtype=torch.float32, hidden=D.hidden):
    """x ~ N(0,1), W_kv_a ~ N(0, 1/hidden), gain = 1 + 0.1 N(0,1) (the q_norm_w convention),
    caches ~ N(0,1) so untouched rows are recognisable."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32)  # noqa: E731
    x = rn(B, Sq, hidden)
    W = rn(hidden, D.kv_rank + D.rope) / math.sqrt(hidden)
    gain = 1.0 + 0.1 * rn(D.kv_rank)
    ck = rn(B, rows, D.kv_rank)
    pe = rn(B, rows, D.rope)
    return [t.to(dtype) for t in (x, W, gain, ck, pe)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_split_wkv_b_is_exact(ext, dtype):
    g = torch.Generator().manual_seed(1)
    wkv_b = torch.randn(D.n_heads, D.nope + D.v, D.kv_rank, generator=g).to(dtype)
    uk, uv = ext.split_wkv_b(gpu(wkv_b), D.nope)
    ruk, ruv = R.split_wkv_b(wkv_b, D.nope)
    assert uk.is_contiguous() and uv.is_contiguous()
    assert torch.equal(uk.cpu(), ruk) and torch.equal(uv.cpu(), ruv)


@pytest.mark.parametrize("B,Sq,rows,start", [(3, 2, 100, 40), (1, 7, 7, 0), (2, 1, 4989, 4988)])
def test_kv_append_matches_oracle(ext, B, Sq, rows, start):
    x, W, gain, ck, pe = kv_inputs(B, Sq, rows, seed=B * 10 + Sq)
    pos = torch.arange(start, start + Sq)
    ck_g, pe_g = gpu(ck), gpu(pe)
    ext.kv_append(gpu(x), gpu(W), gpu(gain), gpu(pos), ck_g, pe_g, start, 1e-6)
    rc, rp = R.kv_append(x, W, gain, pos, ck, pe, start, eps=1e-6)
    got_c, got_p = ck_g.cpu(), pe_g.cpu()
    rows_new = slice(start, start + Sq)
    torch.testing.assert_close(got_c[:, rows_new], rc[:, rows_new], **TOL)
    torch.testing.assert_close(got_p[:, rows_new], rp[:, rows_new], **TOL)
    keep = torch.ones(rows, dtype=torch.bool)
    keep[rows_new] = False
    assert torch.equal(got_c[:, keep], ck[:, keep]) and torch.equal(got_p[:, keep], pe[:, keep])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_kv_append_16bit(ext, dtype):
    B, Sq, rows, start = 2, 3, 50, 10
    x, W, gain, ck, pe = kv_inputs(B, Sq, rows, seed=5, dtype=dtype)
    pos = torch.arange(start, start + Sq)
    ck_g, pe_g = gpu(ck), gpu(pe)
    ext.kv_append(gpu(x), gpu(W), gpu(gain), gpu(pos), ck_g, pe_g, start, 1e-6)
    f = lambda t: t.float()  # noqa: E731
    rc, rp = R.kv_append(f(x), f(W), f(gain), pos, f(ck), f(pe), start, eps=1e-6)
    torch.testing.assert_close(ck_g.cpu().float()[:, start:start + Sq], rc[:, start:start + Sq],
                               **TOL_BF16)
    torch.testing.assert_close(pe_g.cpu().float()[:, start:start + Sq], rp[:, start:start + Sq],
                               **TOL_BF16)


def test_kv_append_then_decode(ext):
    """Decode step end to end: append the new token's cache row, then attend over the
    extended cache; the oracle does the same on the CPU."""
    B, Sk = 2, 300
    inp = R.make_inputs(B, 1, Sk, seed=7)
    _, W, gain, _, _ = kv_inputs(B, 1, Sk, seed=8)
    # the decode token sits at the last position, Sk - 1, both as query and as new key
    pos = inp["positions"]
    assert pos.tolist() == [Sk - 1]
    ck_g, pe_g = gpu(inp["c_kv"]), gpu(inp["pe_cache"])
    ext.kv_append(gpu(inp["x"]), gpu(W), gpu(gain), gpu(pos), ck_g, pe_g, Sk - 1, 1e-6)
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    qa, qr = ext.q_absorbed(gpu(inp["x"]), gpu(inp["W_q_a"]), gpu(inp["q_norm_w"]),
                            gpu(inp["W_q_b"]), gpu(W_uk.contiguous()), gpu(pos), D.nope, D.rope,
                            1e-6)
    out = ext.mla_attention(qa, qr, ck_g, pe_g, gpu(W_uv.contiguous()), SCALE).cpu()
    rc, rp = R.kv_append(inp["x"], W, gain, pos, inp["c_kv"], inp["pe_cache"], Sk - 1)
    ref = R.mla_layer(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], inp["wkv_b"],
                      rc, rp, pos)
    torch.testing.assert_close(out, ref, **TOL)


def test_kv_append_decode_full_size(ext):
    """B=128 decode append (Sq=1) into a 4989-row cache; oracle on three sequences."""
    B, rows, start = 128, 4989, 4988
    x, W, gain, ck, pe = kv_inputs(B, 1, rows, seed=9)
    pos = torch.tensor([start])
    ck_g, pe_g = gpu(ck), gpu(pe)
    ext.kv_append(gpu(x), gpu(W), gpu(gain), gpu(pos), ck_g, pe_g, start, 1e-6)
    pick = [0, 77, 127]
    rc, rp = R.kv_append(x[pick], W, gain, pos, ck[pick], pe[pick], start, eps=1e-6)
    torch.testing.assert_close(ck_g[pick].cpu()[:, start], rc[:, start], **TOL)
    torch.testing.assert_close(pe_g[pick].cpu()[:, start], rp[:, start], **TOL)
    assert torch.equal(ck_g[:, :start].cpu(), ck[:, :start])


@pytest.mark.parametrize("B,Sq", [(1, 1), (4, 3), (128, 1)])
def test_o_proj_matches_oracle(ext, B, Sq):
    g = torch.Generator().manual_seed(B + Sq)
    attn = torch.randn(B, Sq, D.n_heads, D.v, generator=g)
    W_o = torch.randn(D.n_heads * D.v, D.hidden, generator=g) / math.sqrt(D.n_heads * D.v)
    out = ext.o_proj(gpu(attn), gpu(W_o)).cpu()
    pick = list(range(min(B, 3)))
    ref = R.o_proj(attn[pick], W_o)
    assert out.shape == (B, Sq, D.hidden)
    torch.testing.assert_close(out[pick], ref, **TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_o_proj_16bit_b128(ext, monkeypatch, dtype):
    """B=128 decode: the weight-streaming plan (4 K splits, summed by the reduction that
    also rounds to the storage format), every row against the oracle and against the
    tiled engine (MLA_WGEMM=0)."""
    g = torch.Generator().manual_seed(5)
    attn = torch.randn(128, 1, D.n_heads, D.v, generator=g).to(dtype)
    W_o = (torch.randn(D.n_heads * D.v, D.hidden, generator=g) /
           math.sqrt(D.n_heads * D.v)).to(dtype)
    out = ext.o_proj(gpu(attn), gpu(W_o)).cpu().float()
    ref = R.o_proj(attn.float(), W_o.float())
    torch.testing.assert_close(out, ref, **TOL_BF16)
    monkeypatch.setenv("MLA_WGEMM", "0")
    tiled = ext.o_proj(gpu(attn), gpu(W_o)).cpu().float()
    torch.testing.assert_close(out, tiled, **TOL_BF16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_o_proj_16bit(ext, dtype):
    g = torch.Generator().manual_seed(3)
    attn = torch.randn(4, 2, D.n_heads, D.v, generator=g).to(dtype)
    W_o = (torch.randn(D.n_heads * D.v, D.hidden, generator=g) /
           math.sqrt(D.n_heads * D.v)).to(dtype)
    out = ext.o_proj(gpu(attn), gpu(W_o))
    assert out.dtype == dtype
    ref = R.o_proj(attn.float(), W_o.float())
    torch.testing.assert_close(out.cpu().float(), ref, **TOL_BF16)
