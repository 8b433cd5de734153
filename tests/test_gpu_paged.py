"""GPU parity of the ragged, paged KV cache path against the CPU oracle
(``oracle/mla_ref.py``: ``mla_attention_paged``, ``prepare_q_ragged``, ``kv_append_paged``,
pinned in ``tests/test_oracle.py``).

Pools are shuffled (a sequence's pages are scattered through the pool, interleaved with
other sequences' pages and unused ones), lengths are ragged and not multiples of the page
or tile sizes.  Tolerances: fp32 rtol/atol 1e-4; 16-bit attn_cases.tol (bf16 rtol 2e-2,
atol 2e-3 on small outputs) against the fp32 oracle on the rounded inputs, with queries of
the layer's spread; a paged cache laid out like the dense one must give the dense result
bit for bit.  mla_attention_paged runs the fused 3a+3b+3c kernels at the DeepSeek-V3
widths (the block table read per key block, the key chunks of a ragged batch balanced by a
device-built work list); MLA_ATTENTION_PATH=split selects the per-step kernels, and both
paths are checked.
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
TOL = dict(rtol=1e-4, atol=1e-4)


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU (torch.cuda.is_available() is False)")
    import mla_custom_cuda  # noqa: F401  (fails loudly if the extension is not built)
    return mla_custom_cuda


def gpu(t):
    return t.to(DEV)


PATHS = pytest.mark.parametrize("path", ["fused", "split"])


def set_path(monkeypatch, path):
    if path == "split":
        monkeypatch.setenv("MLA_ATTENTION_PATH", "split")
    else:
        monkeypatch.delenv("MLA_ATTENTION_PATH", raising=False)


def paged_inputs(B, Sq, lens, page, max_pages, seed, dtype=torch.float32, spare=5):
    """Queries ~ N(0,1); a shuffled pool of B*max_pages + spare pages ~ N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32).to(dtype)  # noqa: E731
    n_pages = B * max_pages + spare
    table = torch.randperm(n_pages, generator=g)[:B * max_pages].reshape(B, max_pages).int()
    qa = rn(B, Sq, D.n_heads, D.kv_rank)
    qr = rn(B, Sq, D.n_heads, D.rope)
    ck = rn(n_pages, page, D.kv_rank)
    pe = rn(n_pages, page, D.rope)
    wuv = rn(D.n_heads, D.v, D.kv_rank)
    return qa, qr, ck, pe, table, torch.tensor(lens, dtype=torch.int32), wuv


@PATHS
@pytest.mark.parametrize("page,lens,causal,Sq", [
    (64, [640, 1, 333, 65], False, 1),
    (128, [1000, 129, 500], False, 1),
    (64, [200, 77, 640], True, 4),
    (192, [576, 300], True, 2),
    (64, [700, 1, 333, 65, 1200, 128], False, 1),
    (128, [300, 513, 900, 64], True, 2),
])
def test_paged_attention_matches_oracle(ext, monkeypatch, path, page, lens, causal, Sq):
    set_path(monkeypatch, path)
    B = len(lens)
    max_pages = -(-max(lens) // page)
    qa, qr, ck, pe, table, sl, wuv = paged_inputs(B, Sq, lens, page, max_pages, seed=page + B)
    out = ext.mla_attention_paged(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(table), gpu(sl),
                                  gpu(wuv), SCALE, causal).cpu()
    ref = R.mla_attention_paged(qa, qr, ck, pe, table, sl, wuv, SCALE, causal)
    torch.testing.assert_close(out, ref, **TOL)


@PATHS
def test_paged_equals_dense_bitwise(ext, monkeypatch, path):
    """Full lengths and pages laid out in sequence order: the dense cache gives the same
    answer bit for bit on either path.  The paged fused pass always runs the 64-row kernel
    (its work list is built on the device) and then the merge kernel and the 3d GEMM, so
    the dense call is pinned to those for the bitwise check; the dense call's own choice at
    this batch (the fp32 key-split waves, 3d with the merge folded in) agrees to rounding."""
    set_path(monkeypatch, path)
    B, Sk, page = 3, 4992, 64
    g = torch.Generator().manual_seed(31)
    qa = torch.randn(B, 1, D.n_heads, D.kv_rank, generator=g)
    qr = torch.randn(B, 1, D.n_heads, D.rope, generator=g)
    ck = torch.randn(B, Sk, D.kv_rank, generator=g)
    pe = torch.randn(B, Sk, D.rope, generator=g)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g)
    mp = Sk // page
    table = torch.arange(B * mp, dtype=torch.int32).reshape(B, mp)
    sl = torch.full((B,), Sk, dtype=torch.int32)
    own = ext.mla_attention(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(wuv), SCALE)
    monkeypatch.setenv("MLA_FLASH32_WAVE", "0")
    monkeypatch.setenv("MLA_OUT_SMALL", "0")
    dense = ext.mla_attention(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(wuv), SCALE)
    paged = ext.mla_attention_paged(gpu(qa), gpu(qr), gpu(ck.reshape(-1, page, D.kv_rank)),
                                    gpu(pe.reshape(-1, page, D.rope)), gpu(table), gpu(sl),
                                    gpu(wuv), SCALE)
    assert torch.equal(dense.cpu(), paged.cpu())
    torch.testing.assert_close(own.cpu(), paged.cpu(), **TOL)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
def test_paged_balanced_work_list(ext, dtype):
    """One long sequence among short ones: the fused pass's work list cuts the long one into
    many key chunks (merged per row) while the short ones are single chunks written
    directly; every row against the oracle."""
    lens, page = [4989, 1, 2, 3, 100, 64, 65, 700], 64
    B = len(lens)
    max_pages = -(-max(lens) // page)
    qa, qr, ck, pe, table, sl, wuv = paged_inputs(B, 1, lens, page, max_pages, seed=77)
    qa, qr, wuv = qa * C.LAYER_QA_STD, qr * C.LAYER_QR_STD, wuv / math.sqrt(D.kv_rank)
    qa, qr, ck, pe, wuv = [t.to(dtype) for t in (qa, qr, ck, pe, wuv)]
    out = ext.mla_attention_paged(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(table), gpu(sl),
                                  gpu(wuv), SCALE).float().cpu()
    f = lambda t: t.float()  # noqa: E731
    ref = R.mla_attention_paged(f(qa), f(qr), f(ck), f(pe), table, sl, f(wuv), SCALE)
    torch.testing.assert_close(out, ref, **C.tol(dtype, ref))


@pytest.mark.parametrize("uniform", [False, True], ids=["ragged", "equal"])
def test_paged_work_list_many_sequences(ext, uniform):
    """More sequences than the work-list kernel has threads (B = 300: two per thread), with
    ragged lengths against the oracle on every sequence, and with equal lengths bit for bit
    against the dense call."""
    B, page, max_pages = 300, 64, 4
    g = torch.Generator().manual_seed(300)
    lens = (torch.full((B,), 200, dtype=torch.int32) if uniform
            else torch.randint(1, 257, (B,), generator=g, dtype=torch.int32))
    qa, qr, ck, pe, table, _, wuv = paged_inputs(B, 1, [1] * B, page, max_pages, seed=301)
    qa, qr = qa / math.sqrt(D.kv_rank), qr / math.sqrt(D.kv_rank)
    out = ext.mla_attention_paged(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(table), gpu(lens),
                                  gpu(wuv), SCALE).cpu()
    if uniform:
        gather = lambda pool: torch.stack([R.gather_pages(pool, table[b], 200)  # noqa: E731
                                           for b in range(B)])
        dense = ext.mla_attention(gpu(qa), gpu(qr), gpu(gather(ck)), gpu(gather(pe)), gpu(wuv),
                                  SCALE).cpu()
        assert torch.equal(out, dense)
    else:
        ref = R.mla_attention_paged(qa, qr, ck, pe, table, lens, wuv, SCALE)
        torch.testing.assert_close(out, ref, **TOL)


def test_paged_equal_short_lengths_equal_dense(ext, monkeypatch):
    """Every sequence the same length L below the pool's capacity: the work list takes the
    dense plan for L, so the result equals the dense call on [B, L] bit for bit (the dense
    call pinned to the paged pass's 64-row kernel, merge kernel and 3d GEMM; its own choice
    here, the fp32 key-split waves and 3d with the merge folded in, agrees to rounding)."""
    B, L, page, max_pages = 3, 3000, 64, 78
    g = torch.Generator().manual_seed(8)
    qa = torch.randn(B, 1, D.n_heads, D.kv_rank, generator=g)
    qr = torch.randn(B, 1, D.n_heads, D.rope, generator=g)
    ck = torch.randn(B * max_pages, page, D.kv_rank, generator=g)
    pe = torch.randn(B * max_pages, page, D.rope, generator=g)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g)
    table = torch.arange(B * max_pages, dtype=torch.int32).reshape(B, max_pages)
    sl = torch.full((B,), L, dtype=torch.int32)
    dense_ck = ck.reshape(B, max_pages * page, D.kv_rank)[:, :L].contiguous()
    dense_pe = pe.reshape(B, max_pages * page, D.rope)[:, :L].contiguous()
    own = ext.mla_attention(gpu(qa), gpu(qr), gpu(dense_ck), gpu(dense_pe), gpu(wuv), SCALE)
    monkeypatch.setenv("MLA_FLASH32_WAVE", "0")
    monkeypatch.setenv("MLA_OUT_SMALL", "0")
    dense = ext.mla_attention(gpu(qa), gpu(qr), gpu(dense_ck), gpu(dense_pe), gpu(wuv), SCALE)
    paged = ext.mla_attention_paged(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(table), gpu(sl),
                                    gpu(wuv), SCALE)
    assert torch.equal(dense.cpu(), paged.cpu())
    torch.testing.assert_close(own.cpu(), paged.cpu(), **TOL)


@PATHS
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_paged_attention_16bit(ext, monkeypatch, path, dtype):
    """16-bit storage with the layer's spread (queries as tests/attn_cases.py draws them,
    W_uv ~ N(0, 1/kv_rank)), at the 16-bit tolerance of attn_cases.tol."""
    set_path(monkeypatch, path)
    lens, page = [700, 64, 1], 64
    qa, qr, ck, pe, table, sl, wuv = paged_inputs(3, 1, lens, page, 11, seed=9)
    s = 1 / math.sqrt(D.kv_rank)
    qa, qr, ck, pe, wuv = [t.to(dtype) for t in (qa * C.LAYER_QA_STD, qr * C.LAYER_QR_STD, ck,
                                                 pe, wuv * s)]
    out = ext.mla_attention_paged(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(table), gpu(sl),
                                  gpu(wuv), SCALE).float().cpu()
    f = lambda t: t.float()  # noqa: E731
    ref = R.mla_attention_paged(f(qa), f(qr), f(ck), f(pe), table, sl, f(wuv), SCALE)
    torch.testing.assert_close(out, ref, **C.tol(dtype, ref))


def test_q_absorbed_per_sequence_positions(ext):
    inp = R.make_inputs(3, 2, 8, seed=4)
    pos = torch.tensor([[10, 11], [4987, 4988], [0, 1]])
    W_uk = R.split_wkv_b(inp["wkv_b"], D.nope)[0].contiguous()
    qa, qr = ext.q_absorbed(gpu(inp["x"]), gpu(inp["W_q_a"]), gpu(inp["q_norm_w"]),
                            gpu(inp["W_q_b"]), gpu(W_uk), gpu(pos), D.nope, D.rope, 1e-6)
    rqa, rqr = R.prepare_q_ragged(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], W_uk,
                                  pos, D.nope, D.rope)
    torch.testing.assert_close(qa.cpu(), rqa, **TOL)
    torch.testing.assert_close(qr.cpu(), rqr, **TOL)


def test_paged_decode_step_end_to_end(ext):
    """One decode step of a ragged batch: append each sequence's new token at its own slot,
    project its query at its own position, attend over the paged cache."""
    B, page, max_pages = 3, 64, 6
    lens = [300, 64, 129]                        # keys after the append
    inp = R.make_inputs(B, 1, 8, seed=12)
    g = torch.Generator().manual_seed(13)
    n_pages = B * max_pages + 3
    table = torch.randperm(n_pages, generator=g)[:B * max_pages].reshape(B, max_pages).int()
    ck = torch.randn(n_pages, page, D.kv_rank, generator=g)
    pe = torch.randn(n_pages, page, D.rope, generator=g)
    W_kv = torch.randn(D.hidden, D.kv_rank + D.rope, generator=g) / math.sqrt(D.hidden)
    gain = 1.0 + 0.1 * torch.randn(D.kv_rank, generator=g)
    pos = torch.tensor([[n - 1] for n in lens])  # the new token's slot = its position
    sl = torch.tensor(lens, dtype=torch.int32)
    ck_g, pe_g = gpu(ck), gpu(pe)
    ext.kv_append_paged(gpu(inp["x"]), gpu(W_kv), gpu(gain), gpu(pos), gpu(table), ck_g, pe_g,
                        1e-6)
    rc, rp = R.kv_append_paged(inp["x"], W_kv, gain, pos, table, ck, pe)
    torch.testing.assert_close(ck_g.cpu(), rc, **TOL)
    torch.testing.assert_close(pe_g.cpu(), rp, **TOL)
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    qa, qr = ext.q_absorbed(gpu(inp["x"]), gpu(inp["W_q_a"]), gpu(inp["q_norm_w"]),
                            gpu(inp["W_q_b"]), gpu(W_uk.contiguous()), gpu(pos), D.nope, D.rope,
                            1e-6)
    out = ext.mla_attention_paged(qa, qr, ck_g, pe_g, gpu(table), gpu(sl),
                                  gpu(W_uv.contiguous()), SCALE).cpu()
    rqa, rqr = R.prepare_q_ragged(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                  W_uk, pos, D.nope, D.rope)
    ref = R.mla_attention_paged(rqa, rqr, rc, rp, table, sl, W_uv, SCALE)
    torch.testing.assert_close(out, ref, **TOL)


@PATHS
def test_paged_attention_full_size_ragged(ext, monkeypatch, path):
    """B=128 decode over a shuffled 64-key-page pool, lengths ragged in [1, 4989]; every
    sequence against the oracle (a dropped or doubled work-list item would leave some
    sequence's rows wrong)."""
    set_path(monkeypatch, path)
    B, page, max_pages = 128, 64, 78                  # 78 * 64 = 4992 >= 4989
    g = torch.Generator().manual_seed(41)
    lens = torch.randint(1, 4990, (B,), generator=g, dtype=torch.int32)
    lens[0], lens[1] = 4989, 1
    qa, qr, ck, pe, table, _, wuv = paged_inputs(B, 1, [1] * B, page, max_pages, seed=42)
    qa = qa * C.LAYER_QA_STD
    qr = qr * C.LAYER_QR_STD
    out = ext.mla_attention_paged(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(table), gpu(lens),
                                  gpu(wuv), SCALE).cpu()
    assert torch.isfinite(out).all()
    ref = R.mla_attention_paged(qa, qr, ck, pe, table, lens, wuv, SCALE)
    torch.testing.assert_close(out, ref, **TOL)
