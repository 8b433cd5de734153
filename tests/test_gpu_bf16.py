"""GPU parity of the bf16 path (bf16 storage, fp32 accumulation on
bf16 MFMA).

Per step, the oracle runs in fp32 on the very bf16 values the kernel reads (and, where the
kernel rounds an fp32 operand to bf16 before its MFMA -- q_raw in 2c, p*alpha in 3c, ctx in
3d -- on the rounded operand), so each step is held to fp32-accumulation accuracy.  The
whole layer is compared with the fp32 oracle on the bf16-rounded inputs at the bf16
tolerance of tests/attn_cases.py: rtol 2e-2, atol 2e-3 on the layer's outputs (standard
deviation ~0.03 at Sk = 4989).
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
BF = torch.bfloat16


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


def gpu(t):
    return t.to(DEV)


def rb(t):
    """Round to bf16 and back (what the kernel does to an fp32 MFMA operand)."""
    return t.to(BF).float()


@pytest.mark.parametrize("M,N,K", [(128, 1536, 7168), (1, 24576, 1536), (40, 200, 72)])
def test_gemm_bf16(ext, M, N, K):
    g = torch.Generator().manual_seed(M + N)
    A = torch.randn(M, K, generator=g).to(BF)
    W = (torch.randn(K, N, generator=g) / math.sqrt(K)).to(BF)
    got = ext.gemm(gpu(A), gpu(W)).cpu()
    assert got.dtype == torch.float32
    ref = (A.double() @ W.double()).float()
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dt", [BF, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("M,N,K,plan", [
    (128, 1536, 7168, "64,8"),      # 2a1 at B = 128
    (128, 24576, 1536, "128,1"),    # 2a2 at B = 128
    (40, 256, 192, "128,1"),        # rows off the 128-row tile
    (130, 128, 128, "64,2"),        # two row tiles, the second of 2 rows
    (7, 128, 320, "128,3"),         # slices 2, 2, 1 over the splits
    (1, 576, 7168, "64,16"),        # the KV projection's shape at B = 1
    (128, 64, 4096, "64,64"),       # one slice per split
    (128, 512, 128, "256,1,3"),     # 256-column tiles (2c's plan), two slices
    (40, 768, 192, "256,2,3"),      # 256-column tiles, rows off the tile, split
])
def test_weight_streaming_gemm(ext, monkeypatch, dt, M, N, K, plan):
    """The weight-streaming engine (forced by MLA_WGEMM_PLAN) against the float64 product
    of the same 16-bit values, and against the tiled engine (MLA_WGEMM=0)."""
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g).to(dt)
    W = (torch.randn(K, N, generator=g) / math.sqrt(K)).to(dt)
    monkeypatch.setenv("MLA_WGEMM_PLAN", f"{M},{N},{K},1={plan}")
    got = ext.gemm(gpu(A), gpu(W)).cpu()
    ref = (A.double() @ W.double()).float()
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)
    monkeypatch.setenv("MLA_WGEMM", "0")
    tiled = ext.gemm(gpu(A), gpu(W)).cpu()
    torch.testing.assert_close(got, tiled, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dt", [BF, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("B,Sq,per_seq", [(2, 3, False), (5, 1, True), (128, 1, False),
                                           (65, 2, False)])
def test_q_absorbed_fused_epilogue(ext, monkeypatch, dt, B, Sq, per_seq):
    """2a2 on the weight-streaming engine with its fused epilogues gives the same bits as
    the separate launches on the same plan, and matches the fp32 oracle; positions shared
    by the batch (up to 4988) or per sequence.  Three forms: the default, where 2a2 also
    rotates q_rope (2b) and runs 2c on each head's q_nope tile; MLA_QUP_ABSORB=0, where it
    writes q_nope for the 2c launch; MLA_QUP_FUSE=0, 2a2 + the 2b launch + 2c."""
    inp = R.make_inputs(B, Sq, 4989, seed=B + Sq, dtype=dt)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    pos = inp["positions"]
    if per_seq:
        pos = torch.tensor([[4988 - 97 * b] for b in range(B)]) if Sq == 1 else pos
    args = [gpu(inp[k]) for k in ("x", "W_q_a", "q_norm_w", "W_q_b")] + [gpu(W_uk.contiguous()),
                                                                        gpu(pos)]
    M, N = B * Sq, D.n_heads * D.qk_head
    monkeypatch.setenv("MLA_WGEMM_PLAN", f"{M},{N},{D.q_lora},1=128,1")
    qa, qr = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    monkeypatch.setenv("MLA_QUP_ABSORB", "0")
    qa1, qr1 = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    monkeypatch.setenv("MLA_QUP_FUSE", "0")
    qa0, qr0 = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    assert qa.dtype == dt and qr.dtype == dt
    assert torch.equal(qa1, qa0) and torch.equal(qr1, qr0)
    assert torch.equal(qa, qa0) and torch.equal(qr, qr0)
    f32 = {k: (v.float() if v.is_floating_point() else v) for k, v in inp.items()}
    prep = R.prepare_q_ragged if per_seq else R.prepare_q_mla_absorbed
    rqa, rqr = prep(f32["x"], f32["W_q_a"], f32["q_norm_w"], f32["W_q_b"], W_uk.float(), pos,
                    D.nope, D.rope)
    torch.testing.assert_close(qa.float(), rqa, **C.tol(dt, rqa))
    torch.testing.assert_close(qr.float(), rqr, **C.tol(dt, rqr))


def test_rmsnorm_rope_bf16(ext):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, 1536, generator=g)
    w = (1 + 0.1 * torch.randn(1536, generator=g)).to(BF)
    got = ext.rmsnorm(gpu(x), gpu(w), 1e-6).cpu()
    assert got.dtype == BF
    ref = R.step_norm(x, w.float(), 1e-6, BF)
    torch.testing.assert_close(got.float(), ref.float(), rtol=1e-2, atol=1e-2)
    q_raw = torch.randn(8, D.n_heads * D.qk_head, generator=g)
    pos = torch.tensor([4988])
    got = ext.rope(gpu(q_raw), gpu(pos), 8, 1, D.n_heads, D.nope, D.rope, BF).cpu()
    ref = R.step_rope(q_raw, pos, R.rope_inv_freq(D.rope), 8, 1, D.n_heads, D.nope, D.rope, BF)
    assert got.dtype == BF
    torch.testing.assert_close(got.float(), ref.float(), rtol=1e-2, atol=1e-2)


def test_absorb_bf16(ext):
    g = torch.Generator().manual_seed(4)
    B, Sq = 16, 1
    q_raw = torch.randn(B * Sq, D.n_heads * D.qk_head, generator=g)
    W_uk = (torch.randn(D.n_heads, D.nope, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)).to(BF)
    got = ext.absorb(gpu(q_raw), gpu(W_uk), B, Sq, D.rope).cpu()
    assert got.dtype == BF
    ref = R.step_absorb(rb(q_raw).double(), W_uk.double(), B, Sq, D.nope, torch.float64)
    torch.testing.assert_close(got.float(), ref.float(), rtol=8e-3, atol=8e-3)


@pytest.mark.parametrize("B,Sq,Sk,causal", [(2, 1, 4989, False), (1, 8, 300, True)])
def test_attention_steps_bf16(ext, B, Sq, Sk, causal):
    g = torch.Generator().manual_seed(Sk)
    mk = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(BF)  # noqa: E731
    qa, qr = mk(B, Sq, D.n_heads, D.kv_rank, sc=0.05), mk(B, Sq, D.n_heads, D.rope, sc=0.05)
    ck, pe = mk(B, Sk, D.kv_rank), mk(B, Sk, D.rope)
    wuv = mk(D.n_heads, D.v, D.kv_rank, sc=1 / math.sqrt(D.kv_rank))
    p, m, l = ext.scores(gpu(qa), gpu(qr), gpu(ck), gpu(pe), SCALE, causal)
    rp, rm, rl = R.step_scores(qa.float(), qr.float(), ck.float(), pe.float(), SCALE,
                               R.SCORE_TILE, causal)
    torch.testing.assert_close(m.cpu(), rm, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(l.cpu(), rl, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(p.cpu()[:, :Sk], rp, rtol=1e-4, atol=1e-5)
    alpha, rs = ext.combine(m, l)
    ctx = ext.ctx(p, alpha, gpu(ck), Sq, D.n_heads)
    a = alpha.cpu().repeat_interleave(R.SCORE_TILE, dim=1)[:, :Sk]
    w = rb(p.cpu()[:, :Sk] * a).double().reshape(B, Sq * D.n_heads, Sk)
    rctx = torch.bmm(w, ck.double()).reshape(B, Sq, D.n_heads, -1).float()
    torch.testing.assert_close(ctx.cpu(), rctx, rtol=1e-4, atol=1e-3)
    out = ext.out(ctx, rs, gpu(wuv)).cpu()
    assert out.dtype == BF
    cn = rb(ctx.cpu() / rs.cpu().reshape(B, Sq, D.n_heads, 1))
    rout = torch.einsum("bshr,hdr->bshd", cn.double(), wuv.double()).float()
    torch.testing.assert_close(out.float(), rout, rtol=8e-3, atol=8e-3)


def run_layer(ext, inp, causal=False):
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    g = {k: gpu(v) for k, v in inp.items()}
    qa, qr = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"],
                            gpu(W_uk.contiguous()), g["positions"], D.nope, D.rope, 1e-6)
    out = ext.mla_attention(qa, qr, g["c_kv"], g["pe_cache"], gpu(W_uv.contiguous()), SCALE,
                            causal)
    return qa, qr, out


@pytest.mark.parametrize("B,Sq,Sk", [(4, 1, 4989), (1, 1, 512), (2, 3, 1000)])
def test_layer_bf16_vs_fp32_oracle(ext, B, Sq, Sk):
    inp = R.make_inputs(B, Sq, Sk, seed=0, dtype=BF)
    qa, qr, out = run_layer(ext, inp)
    assert out.dtype == BF and qa.dtype == BF and qr.dtype == BF
    f32 = {k: (v.float() if v.is_floating_point() else v) for k, v in inp.items()}
    ref = R.mla_layer(f32["x"], f32["W_q_a"], f32["q_norm_w"], f32["W_q_b"], f32["wkv_b"],
                      f32["c_kv"], f32["pe_cache"], f32["positions"])
    torch.testing.assert_close(out.float().cpu(), ref, **C.tol(BF, ref))


def test_layer_bf16_cfg4_full_size(ext):
    """bf16 decode at B=128, Sq=1, Sk=4989; every sequence against the fp32 oracle on the
    bf16-rounded inputs at the bf16 tolerance."""
    inp = R.make_inputs(128, 1, 4989, seed=0, dtype=BF)
    qa, qr, out = run_layer(ext, inp)
    assert torch.isfinite(out.float()).all()
    f32 = {k: (v.float() if v.is_floating_point() else v) for k, v in inp.items()}
    ref = R.mla_layer(f32["x"], f32["W_q_a"], f32["q_norm_w"], f32["W_q_b"], f32["wkv_b"],
                      f32["c_kv"], f32["pe_cache"], f32["positions"])
    torch.testing.assert_close(out.float().cpu(), ref, **C.tol(BF, ref))


@pytest.mark.parametrize("dt", [BF, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("B,Sk,plan", [(128, 1000, None), (130, 300, "128,1,4"),
                                       (128, 700, "64,1,3"), (40, 64, "64,1,4")])
def test_out_projection_3d_weight_streaming(ext, monkeypatch, dt, B, Sk, plan):
    """3d from the pass's normalised 16-bit ctx on the weight-streaming engine's NT tiles
    (W_uv rows K-contiguous, G = heads, the output rounded in its epilogue): the same bits
    as the tiled engine (MLA_WGEMM=0), over one and two row tiles and a partial one, and
    the oracle's result at the 16-bit tolerance."""
    g = torch.Generator().manual_seed(B + Sk)
    mk = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(dt)  # noqa: E731
    qa, qr = mk(B, 1, D.n_heads, D.kv_rank, sc=0.05), mk(B, 1, D.n_heads, D.rope, sc=0.05)
    ck, pe = mk(B, Sk, D.kv_rank), mk(B, Sk, D.rope)
    wuv = mk(D.n_heads, D.v, D.kv_rank, sc=1 / math.sqrt(D.kv_rank))
    if plan:
        monkeypatch.setenv("MLA_WGEMM_PLAN", f"{B},{D.v},{D.kv_rank},{D.n_heads}={plan}")
    args = [gpu(t) for t in (qa, qr, ck, pe, wuv)]
    got = ext.mla_attention(*args, SCALE).cpu()
    monkeypatch.setenv("MLA_WGEMM", "0")
    tiled = ext.mla_attention(*args, SCALE).cpu()
    assert got.dtype == dt and torch.equal(got, tiled)
    f = lambda t: t.float()  # noqa: E731
    ref = R.mla_attention_official(f(qa), f(qr), f(ck), f(pe), f(wuv), SCALE)
    torch.testing.assert_close(got.float(), ref, **C.tol(dt, ref))


@pytest.mark.parametrize("dt", [BF, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("B,plan", [(128, "128,1,4"), (130, "64,1,3"), (40, "128,1,3")])
def test_absorb_on_weight_streaming_groups(ext, monkeypatch, dt, B, plan):
    """2c as its own launch from 2a2's 16-bit q_nope (2a2's plan forced to the fused
    epilogue, MLA_QUP_ABSORB=0) forced onto the weight-streaming engine: NN tiles over
    G = heads groups with the output in the storage format give the same bits as the tiled
    engine's 2c, over one, two and a partial row tile."""
    inp = R.make_inputs(B, 1, 64, seed=B, dtype=dt)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    args = [gpu(inp[k]) for k in ("x", "W_q_a", "q_norm_w", "W_q_b")] + [gpu(W_uk.contiguous()),
                                                                        gpu(inp["positions"])]
    monkeypatch.setenv("MLA_QUP_ABSORB", "0")
    up = f"{B},{D.n_heads * D.qk_head},{D.q_lora},1=128,1"   # 2a2 fused: 16-bit q_nope
    monkeypatch.setenv("MLA_WGEMM_PLAN", f"{up};{B},{D.kv_rank},{D.nope},{D.n_heads}={plan}")
    qa, qr = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    monkeypatch.setenv("MLA_WGEMM_PLAN", up)
    qa0, qr0 = (t.cpu() for t in ext.q_absorbed(*args, D.nope, D.rope, 1e-6))
    assert torch.equal(qa, qa0) and torch.equal(qr, qr0)
