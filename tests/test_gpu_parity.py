"""GPU parity: every HIP step and both fused entry points against the CPU oracle.

Runs on a real MI355X only (``-m gpu``).  Inputs are the oracle's seeded CPU tensors
copied to the GPU, so HIP path and oracle see identical values.  Tolerances:

* fp32 final output [B,Sq,H,v]: rtol 1e-4 / atol 1e-4, and for the
  reference's tile-straddling shape sweep also its own criterion: error within 5x the
  fp32-vs-fp64 noise of the same op (check_3d.py:40-44);
* per-step fp32 intermediates: rtol/atol 1e-4 on O(1) quantities, 1e-5 on softmax factors.

Layer tests compare every sequence with the oracle, the headline size (B=128, Sk=4989)
included; the long-context causal shape compares its whole Q path and all 512 query rows
of the attention, each against the oracle on exactly the keys it sees.
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


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU (torch.cuda.is_available() is False)")
    import mla_custom_cuda  # noqa: F401  (fails loudly if the extension is not built)
    return mla_custom_cuda


def gpu(t):
    return t.to(DEV)


def attn_inputs(B, Sq, Sk, seed=0, dims=D, dtype=torch.float32):
    """q_absorbed/q_rope/c_kv/pe/W_uv ~ N(0,1) as in check_3d.py:27-32 (CPU generator)."""
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32).to(dtype)  # noqa: E731
    return (mk(B, Sq, dims.n_heads, dims.kv_rank), mk(B, Sq, dims.n_heads, dims.rope),
            mk(B, Sk, dims.kv_rank), mk(B, Sk, dims.rope), mk(dims.n_heads, dims.v, dims.kv_rank))


# ------------------------------------------------------------------ per step


@pytest.mark.parametrize("M,N,K", [(128, 1536, 7168), (1, 1536, 7168), (7, 24576, 1536),
                                   (130, 200, 68), (33, 64, 4)])
def test_gemm(ext, M, N, K):
    g = torch.Generator().manual_seed(M * 7 + N)
    A = torch.randn(M, K, generator=g)
    W = torch.randn(K, N, generator=g) / math.sqrt(K)
    got = ext.gemm(gpu(A), gpu(W)).cpu()
    ref = (A.double() @ W.double()).float()
    torch.testing.assert_close(got, ref, **TOL)


@pytest.mark.parametrize("M,N,K", [(1, 1536, 7168), (3, 1000, 300), (5, 260, 4100),
                                   (2, 4, 64), (8, 24576, 1536), (4, 512, 36), (6, 260, 100)])
def test_gemm_small_m(ext, M, N, K):
    """Decode-sized products (M <= 8, fp32): a tile mostly past M, ragged column tiles, K
    splits with a short last chunk, K below one slice."""
    g = torch.Generator().manual_seed(M * 1000 + K)
    A = torch.randn(M, K, generator=g)
    W = torch.randn(K, N, generator=g) / math.sqrt(K)
    got = ext.gemm(gpu(A), gpu(W)).cpu()
    ref = (A.double() @ W.double()).float()
    torch.testing.assert_close(got, ref, **TOL)


@pytest.mark.parametrize("plan", ["64,64,1,3", "64,64,3,5", "128,128,1,7", "32,128,2,2"])
def test_gemm_persistent_plans(ext, monkeypatch, plan):
    """Forced persistent-grid plans (bm, bn, split, tiles per workgroup) of the 2a1 shape:
    workgroups with unequal tile counts, a split whose last chunk is one slice short, and
    slice streams of odd length (padded with a zero slice) all give the float64 product."""
    M, N, K = 128, 1536, 7168
    monkeypatch.setenv("MLA_GEMM_PLAN", f"{M},{N},{K},1={plan}")
    g = torch.Generator().manual_seed(5)
    A = torch.randn(M, K, generator=g)
    W = torch.randn(K, N, generator=g) / math.sqrt(K)
    got = ext.gemm(gpu(A), gpu(W)).cpu()
    ref = (A.double() @ W.double()).float()
    torch.testing.assert_close(got, ref, **TOL)


@pytest.mark.parametrize("M", [1, 128, 300])
def test_rmsnorm(ext, M):
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, 1536, generator=g) * 0.3
    w = 1.0 + 0.1 * torch.randn(1536, generator=g)
    got = ext.rmsnorm(gpu(x), gpu(w), 1e-6).cpu()
    torch.testing.assert_close(got, R.step_norm(x, w, 1e-6, torch.float32), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("B,Sq,pos0", [(2, 1, 4988), (3, 4, 0), (1, 7, 65500)])
def test_rope(ext, B, Sq, pos0):
    g = torch.Generator().manual_seed(B + Sq)
    q_raw = torch.randn(B * Sq, D.n_heads * D.qk_head, generator=g)
    pos = torch.arange(pos0, pos0 + Sq)
    got = ext.rope(gpu(q_raw), gpu(pos), B, Sq, D.n_heads, D.nope, D.rope, torch.float32).cpu()
    ref = R.step_rope(q_raw, pos, R.rope_inv_freq(D.rope), B, Sq, D.n_heads, D.nope, D.rope,
                      torch.float32)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("B,Sq", [(1, 1), (128, 1), (4, 33)])
def test_absorb(ext, B, Sq):
    g = torch.Generator().manual_seed(B * Sq)
    q_raw = torch.randn(B * Sq, D.n_heads * D.qk_head, generator=g)
    W_uk = torch.randn(D.n_heads, D.nope, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)
    got = ext.absorb(gpu(q_raw), gpu(W_uk), B, Sq, D.rope).cpu()
    ref = R.step_absorb(q_raw.double(), W_uk.double(), B, Sq, D.nope, torch.float64).float()
    torch.testing.assert_close(got, ref, **TOL)


@pytest.mark.parametrize("B,Sq,Sk,causal", [(1, 1, 512, False), (2, 3, 1000, False),
                                            (1, 1, 4989, False), (2, 4, 300, True),
                                            (1, 2, 129, True)])
def test_scores_combine_ctx_out(ext, B, Sq, Sk, causal):
    qa, qr, ck, pe, wuv = attn_inputs(B, Sq, Sk, seed=Sk)
    qa, qr = qa * 0.05, qr * 0.05  # keep scores O(1): p is compared elementwise
    p, m, l = ext.scores(gpu(qa), gpu(qr), gpu(ck), gpu(pe), SCALE, causal)
    rp, rm, rl = R.step_scores(qa, qr, ck, pe, SCALE, R.SCORE_TILE, causal)
    P = rm.shape[1]
    assert p.shape[1] == ext.score_ld(Sk) and m.shape == (B * Sq * D.n_heads, P)
    torch.testing.assert_close(m.cpu(), rm, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(l.cpu(), rl, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(p.cpu()[:, :Sk], rp, rtol=1e-4, atol=1e-5)
    assert (p.cpu()[:, Sk:] == 0).all(), "score row padding must be zero"
    # 3b on the GPU's partials
    alpha, rs = ext.combine(m, l)
    ralpha, rrs = R.step_combine(m.cpu(), l.cpu())
    torch.testing.assert_close(alpha.cpu(), ralpha, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(rs.cpu(), rrs, rtol=1e-5, atol=1e-5)
    # 3c on the GPU's p / alpha
    ctx = ext.ctx(p, alpha, gpu(ck), Sq, D.n_heads)
    rctx = R.step_ctx(p.cpu()[:, :Sk].double(), alpha.cpu().double(), ck.double(), B, Sq,
                      D.n_heads).float()
    torch.testing.assert_close(ctx.cpu(), rctx, rtol=1e-4, atol=1e-3)
    # 3d on the GPU's ctx / row_sum
    out = ext.out(ctx, rs, gpu(wuv))
    rout = R.step_out(ctx.cpu().double(), rs.cpu().double(), wuv.double(), torch.float64).float()
    torch.testing.assert_close(out.cpu(), rout, **TOL)


# ------------------------------------------------------------------ fused attention

CHECK_3D_SHAPES = [(1, 1, 32), (3, 7, 40), (1, 64, 64), (1, 65, 48), (2, 33, 96), (5, 13, 71),
                   (1, 1, 4096), (1, 1, 4999), (2, 3, 1000), (1, 1, 16384), (1, 2, 8191)]


@pytest.mark.parametrize("B,Sq,Sk", CHECK_3D_SHAPES)
def test_attention_check3d_shapes(ext, B, Sq, Sk):
    """The reference's tile-boundary sweep (check_3d.py:20-44): N(0,1) inputs, error
    within 5x the fp32-vs-fp64 noise of the same op."""
    qa, qr, ck, pe, wuv = attn_inputs(B, Sq, Sk, seed=0)
    out = ext.mla_attention(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(wuv), SCALE).cpu()
    assert out.shape == (B, Sq, D.n_heads, D.v) and out.dtype == torch.float32
    ref32 = R.mla_attention_official(qa, qr, ck, pe, wuv, SCALE)
    ref64 = R.mla_attention_official(qa.double(), qr.double(), ck.double(), pe.double(),
                                     wuv.double(), SCALE)
    err = (out.double() - ref64).abs().max().item()
    noise = (ref32.double() - ref64).abs().max().item()
    assert err < 5 * max(noise, 1e-6), f"err {err:.3e} vs fp32 noise {noise:.3e}"


@pytest.mark.parametrize("Sk,path", [(64, "plain"), (16384, "split-K")])
def test_attention_check_dtypes_fp32(ext, Sk, path):
    """check_dtypes.py:23-38, fp32 row: relative-to-max error < 1e-5, output dtype kept."""
    qa, qr, ck, pe, wuv = attn_inputs(1, 1, Sk, seed=0)
    out = ext.mla_attention(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(wuv), SCALE).cpu()
    ref = R.mla_attention_official(qa.double(), qr.double(), ck.double(), pe.double(),
                                   wuv.double(), SCALE)
    assert out.dtype == torch.float32
    rel = ((out.double() - ref).abs().max() / ref.abs().max()).item()
    assert rel < 1e-5, rel


@pytest.mark.parametrize("B,Sq,Sk", [(2, 16, 300), (1, 128, 1024), (3, 5, 5)])
def test_attention_causal(ext, B, Sq, Sk):
    qa, qr, ck, pe, wuv = attn_inputs(B, Sq, Sk, seed=3)
    out = ext.mla_attention(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(wuv), SCALE, True).cpu()
    ref = R.mla_attention_official(qa.double(), qr.double(), ck.double(), pe.double(),
                                   wuv.double(), SCALE, causal=True).float()
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=2e-4)


def test_attention_causal_single_query_equals_noncausal(ext):
    qa, qr, ck, pe, wuv = attn_inputs(2, 1, 700, seed=4)
    args = [gpu(t) for t in (qa, qr, ck, pe, wuv)]
    a = ext.mla_attention(*args, SCALE, True)
    b = ext.mla_attention(*args, SCALE, False)
    assert torch.equal(a, b)


def test_attention_deterministic(ext):
    qa, qr, ck, pe, wuv = attn_inputs(1, 1, 16384, seed=5)
    args = [gpu(t) for t in (qa, qr, ck, pe, wuv)]
    a = ext.mla_attention(*args, SCALE)
    b = ext.mla_attention(*args, SCALE)
    assert torch.equal(a, b), "split-K must be order-deterministic"


# ------------------------------------------------------------------ fused Q path + layer


def run_layer(ext, inp, causal=False):
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    g = {k: gpu(v) for k, v in inp.items()}
    qa, qr = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"],
                            gpu(W_uk.contiguous()), g["positions"], D.nope, D.rope, 1e-6)
    out = ext.mla_attention(qa, qr, g["c_kv"], g["pe_cache"], gpu(W_uv.contiguous()), SCALE,
                            causal)
    return qa, qr, out


def oracle_layer_rows(inp, batches):
    """Oracle for a subset of sequences (each sequence is independent)."""
    sub = dict(inp)
    for k in ("x", "c_kv", "pe_cache"):
        sub[k] = inp[k][batches]
    W_uk, W_uv = R.split_wkv_b(sub["wkv_b"], D.nope)
    qa, qr = R.prepare_q_mla_absorbed(sub["x"], sub["W_q_a"], sub["q_norm_w"], sub["W_q_b"],
                                      W_uk, sub["positions"], D.nope, D.rope)
    out = R.mla_attention_official(qa, qr, sub["c_kv"], sub["pe_cache"], W_uv, SCALE)
    return qa, qr, out


def test_q_absorbed_cfg1(ext):
    inp = R.make_inputs(1, 1, 512, seed=0)
    qa, qr, out = run_layer(ext, inp)
    rqa, rqr, rout = oracle_layer_rows(inp, [0])
    assert qa.shape == (1, 1, D.n_heads, D.kv_rank) and qr.shape == (1, 1, D.n_heads, D.rope)
    torch.testing.assert_close(qr.cpu(), rqr, **TOL)
    torch.testing.assert_close(qa.cpu(), rqa, **TOL)
    torch.testing.assert_close(out.cpu(), rout, **TOL)


@pytest.mark.parametrize("B", [1, 8, 32])
def test_layer_cfg3_small_batch(ext, B):
    inp = R.make_inputs(B, 1, 4989, seed=0)
    qa, qr, out = run_layer(ext, inp)
    rqa, rqr, rout = oracle_layer_rows(inp, list(range(B)))
    torch.testing.assert_close(qa.cpu(), rqa, **TOL)
    torch.testing.assert_close(qr.cpu(), rqr, **TOL)
    torch.testing.assert_close(out.cpu(), rout, **TOL)


@pytest.mark.parametrize("B,Sq,per_seq", [(1, 1, False), (2, 3, False), (8, 1, True),
                                           (3, 3, False)])
def test_q_absorbed_small_batch_kernel(ext, monkeypatch, B, Sq, per_seq):
    """fp32 decode batches of B*Sq <= 8 rows run 2b and 2c as one VALU kernel
    (q_small_kernel); MLA_Q_SMALL=0 keeps the 2b launch and the MFMA 2c.  q_rope is the
    same to the bit (same sums, angles and rotation); q_absorbed differs only in the order
    of its fp32 sums.  Both match the oracle.  (3, 3) has 9 rows, past the kernel's 8: both
    runs take the launches."""
    inp = R.make_inputs(B, Sq, 4989, seed=B * 10 + Sq)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    pos = inp["positions"]
    if per_seq:
        pos = torch.tensor([[4988 - 131 * b] for b in range(B)])
    args = [gpu(inp[k]) for k in ("x", "W_q_a", "q_norm_w", "W_q_b")] + [gpu(W_uk.contiguous()),
                                                                        gpu(pos)]
    qa, qr = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    monkeypatch.setenv("MLA_Q_SMALL", "0")
    qa0, qr0 = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    assert torch.equal(qr, qr0)
    if B * Sq > 8:
        assert torch.equal(qa, qa0)
    torch.testing.assert_close(qa, qa0, rtol=1e-5, atol=1e-5)
    prep = R.prepare_q_ragged if per_seq else R.prepare_q_mla_absorbed
    rqa, rqr = prep(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], W_uk, pos, D.nope,
                    D.rope)
    torch.testing.assert_close(qa, rqa, **TOL)
    torch.testing.assert_close(qr, rqr, **TOL)


@pytest.mark.parametrize("split", [1, 8])
def test_q_absorbed_small_batch_kernel_split_range(ext, monkeypatch, split):
    """The small-batch 2b + 2c kernel after an unsplit 2a2 (it reads 2a2's output) and
    after the most split partials it holds (8), 2a2's plan forced; against the two-launch
    form and the oracle."""
    B, Sq = 2, 1
    inp = R.make_inputs(B, Sq, 4989, seed=70 + split)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    args = [gpu(inp[k]) for k in ("x", "W_q_a", "q_norm_w", "W_q_b")] + [gpu(W_uk.contiguous()),
                                                                        gpu(inp["positions"])]
    shape = f"{B * Sq},{D.n_heads * D.qk_head},{D.q_lora},1"
    monkeypatch.setenv("MLA_GEMM_PLAN", f"{shape}=32,128,{split}")
    qa, qr = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    monkeypatch.setenv("MLA_Q_SMALL", "0")
    qa0, qr0 = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    assert torch.equal(qr, qr0)
    torch.testing.assert_close(qa, qa0, rtol=1e-5, atol=1e-5)
    rqa, rqr = R.prepare_q_mla_absorbed(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                        W_uk, inp["positions"], D.nope, D.rope)
    torch.testing.assert_close(qa, rqa, **TOL)
    torch.testing.assert_close(qr, rqr, **TOL)


def test_layer_cfg2_full_size(ext):
    """Headline decode shape: B=128, Sq=1, Sk=4989, fp32, full DeepSeek-V3 dims; every
    sequence against the oracle at the north-star tolerance."""
    inp = R.make_inputs(128, 1, 4989, seed=0)
    qa, qr, out = run_layer(ext, inp)
    assert torch.isfinite(out).all()
    rqa, rqr, rout = oracle_layer_rows(inp, list(range(128)))
    torch.testing.assert_close(qa.cpu(), rqa, **TOL)
    torch.testing.assert_close(qr.cpu(), rqr, **TOL)
    torch.testing.assert_close(out.cpu(), rout, **TOL)


def test_layer_cfg5_fused_causal_full_size(ext):
    """The chunked-prefill configuration through the path bench.py times: q_absorbed at
    Sq=128 with positions Sk-128 .. Sk-1, then the fused mla_attention(causal=True), B=4,
    Sk=32768, fp32.  The Q path is compared whole, and so is the attention: all 512
    (sequence, query) rows against the oracle on exactly the keys each query sees (key j
    visible to query s iff j <= Sk - Sq + s).  The oracle runs in blocks of 32 queries:
    queries s0 .. s0+31 over keys [0, Sk - Sq + s0 + 32) are the causal problem of
    R.causal_mask(32, Sk - Sq + s0 + 32), the same visibility rule."""
    B, Sq, Sk = 4, 128, 32768
    inp = R.make_inputs(B, Sq, Sk, seed=0)
    qa, qr, out = run_layer(ext, inp, causal=True)
    assert out.shape == (B, Sq, D.n_heads, D.v) and torch.isfinite(out).all()
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    rqa, rqr = R.prepare_q_mla_absorbed(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                        W_uk, inp["positions"], D.nope, D.rope)
    torch.testing.assert_close(qa.cpu(), rqa, **TOL)
    torch.testing.assert_close(qr.cpu(), rqr, **TOL)
    qa_c, qr_c, out_c = qa.cpu(), qr.cpu(), out.cpu()
    step = 32
    for b in range(B):
        for s0 in range(0, Sq, step):
            lim = Sk - Sq + s0 + step
            ref = R.mla_attention_official(qa_c[b:b + 1, s0:s0 + step],
                                           qr_c[b:b + 1, s0:s0 + step],
                                           inp["c_kv"][b:b + 1, :lim],
                                           inp["pe_cache"][b:b + 1, :lim], W_uv, SCALE,
                                           causal=True)
            torch.testing.assert_close(out_c[b, s0:s0 + step], ref[0], **TOL)


def test_reference_input_convention(ext):
    """The reference's own input scaling (exhaustive_benchmark_suite.py:346-376) at its
    --quick scenario shape (B=64, Sq=2, Sk=512), compared with its suite gate
    (rtol/atol 3e-2, :471) and with the north-star 1e-4."""
    inp = R.make_inputs(64, 2, 512, seed=1)
    inp["x"] = inp["x"] / math.sqrt(D.hidden)
    inp["c_kv"] = inp["c_kv"] / math.sqrt(D.kv_rank)
    inp["pe_cache"] = inp["pe_cache"] / math.sqrt(D.rope)
    inp["wkv_b"] = inp["wkv_b"] * math.sqrt(D.kv_rank) / math.sqrt(D.nope)
    qa, qr, out = run_layer(ext, inp)
    _, _, rout = oracle_layer_rows(inp, list(range(64)))
    torch.testing.assert_close(out.cpu(), rout, rtol=3e-2, atol=3e-2)
    torch.testing.assert_close(out.cpu(), rout, **TOL)


@pytest.mark.parametrize("B,Sq,per_seq,plan", [
    (128, 1, False, None), (130, 1, True, "64,64"), (4, 33, False, "32,128"),
    (4, 128, False, "64,64"), (3, 40, True, "128,32")])
def test_q_absorbed_rope_in_2a2_epilogue(ext, monkeypatch, B, Sq, per_seq, plan):
    """fp32 batches whose 2a2 runs in one K split on tiles of one 32x32 block per wave rotate
    q_rope in 2a2's epilogue (no 2b launch): q_rope and q_absorbed are the same bits as with
    the RoPE launch (MLA_ROPE_EPI=0), and match the oracle; each such tile (forced where the
    planner picks another), full and partial row tiles, positions shared or per sequence."""
    if plan:
        monkeypatch.setenv("MLA_GEMM_PLAN", f"{B * Sq},{D.n_heads * D.qk_head},{D.q_lora},1="
                                            f"{plan},1")
    inp = R.make_inputs(B, Sq, 4989, seed=B + 7 * Sq)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    pos = inp["positions"]
    if per_seq:
        pos = torch.tensor([[4988 - 31 * b - Sq + 1 + s for s in range(Sq)] for b in range(B)])
    args = [gpu(inp[k]) for k in ("x", "W_q_a", "q_norm_w", "W_q_b")] + [gpu(W_uk.contiguous()),
                                                                        gpu(pos)]
    qa, qr = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    monkeypatch.setenv("MLA_ROPE_EPI", "0")
    qa0, qr0 = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    assert torch.equal(qr, qr0) and torch.equal(qa, qa0)
    prep = R.prepare_q_ragged if per_seq else R.prepare_q_mla_absorbed
    rqa, rqr = prep(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], W_uk, pos, D.nope,
                    D.rope)
    torch.testing.assert_close(qa, rqa, **TOL)
    torch.testing.assert_close(qr, rqr, **TOL)


@pytest.mark.parametrize("plan", ["64,64", "32,128", "128,32"])
def test_q_absorbed_rope_epilogue_other_dims(ext, monkeypatch, plan):
    """The fp32 2a2 RoPE epilogue at other widths (6 heads of 64 nope + 32 rope columns, so a
    head's rope part is one 32-column block and tiles cross heads), on each tile it runs on:
    the same bits as the RoPE launch, and the oracle's values."""
    dims = R.MLADims(hidden=256, n_heads=6, q_lora=128, kv_rank=128, nope=64, rope=32, v=64)
    B, Sq = 70, 2
    monkeypatch.setenv("MLA_GEMM_PLAN", f"{B * Sq},{dims.n_heads * dims.qk_head},{dims.q_lora},1="
                                        f"{plan},1")
    inp = R.make_inputs(B, Sq, 300, dims, seed=5)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], dims.nope)
    args = [gpu(inp[k]) for k in ("x", "W_q_a", "q_norm_w", "W_q_b")] + [gpu(W_uk.contiguous()),
                                                                        gpu(inp["positions"])]
    qa, qr = (t.cpu() for t in ext.q_absorbed(*args, dims.nope, dims.rope, 1e-6))
    monkeypatch.setenv("MLA_ROPE_EPI", "0")
    qa0, qr0 = (t.cpu() for t in ext.q_absorbed(*args, dims.nope, dims.rope, 1e-6))
    assert torch.equal(qr, qr0) and torch.equal(qa, qa0)
    rqa, rqr = R.prepare_q_mla_absorbed(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                        W_uk, inp["positions"], dims.nope, dims.rope)
    torch.testing.assert_close(qa, rqa, **TOL)
    torch.testing.assert_close(qr, rqr, **TOL)
