"""GPU parity of the fp16 path: fp16 storage, fp32 accumulation on the gfx950 fp16 MFMAs.

The reference dispatches every step on float16 as well as float32 and float64
(AT_DISPATCH_FLOATING_TYPES_AND_HALF, mla_kernels.cu:674, 726, 739, 1561, 1583, 1610, 1641),
and its dtype check runs the attention in float16 at Sk = 64 (no key split) and Sk = 16384
(split), with randn inputs, against a float64 run of its PyTorch reference: the output
keeps the input dtype and max|out - ref| / max|ref| < 3e-2 (check_dtypes.py:23-38).
`test_attention_f16_like_check_dtypes` mirrors those rows on both attention paths here
(the fused pass and MLA_ATTENTION_PATH=split).

Per step, as for bf16, the oracle runs on the very fp16 values the kernel reads (and on the
rounded operand where a kernel rounds an fp32 operand to fp16 before its MFMA), so each step
is held to fp32-accumulation accuracy; whole layers are compared with the fp32 oracle on
the fp16-rounded inputs.
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
H16 = torch.float16


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


def gpu(t):
    return t.to(DEV)


def rh(t):
    """Round to fp16 and back (what a kernel does to an fp32 MFMA operand)."""
    return t.to(H16).float()


@pytest.mark.parametrize("M,N,K", [(128, 1536, 7168), (1, 24576, 1536), (40, 200, 72)])
def test_gemm_f16(ext, M, N, K):
    g = torch.Generator().manual_seed(M + N + 1)
    A = torch.randn(M, K, generator=g).to(H16)
    W = (torch.randn(K, N, generator=g) / math.sqrt(K)).to(H16)
    got = ext.gemm(gpu(A), gpu(W)).cpu()
    assert got.dtype == torch.float32
    ref = (A.double() @ W.double()).float()
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)


def test_rmsnorm_rope_f16(ext):
    g = torch.Generator().manual_seed(13)
    x = torch.randn(16, 1536, generator=g)
    w = (1 + 0.1 * torch.randn(1536, generator=g)).to(H16)
    got = ext.rmsnorm(gpu(x), gpu(w), 1e-6).cpu()
    assert got.dtype == H16
    ref = R.step_norm(x, w.float(), 1e-6, H16)
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-3, atol=2e-3)
    q_raw = torch.randn(8, D.n_heads * D.qk_head, generator=g)
    pos = torch.tensor([4988])
    got = ext.rope(gpu(q_raw), gpu(pos), 8, 1, D.n_heads, D.nope, D.rope, H16).cpu()
    ref = R.step_rope(q_raw, pos, R.rope_inv_freq(D.rope), 8, 1, D.n_heads, D.nope, D.rope, H16)
    assert got.dtype == H16
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-3, atol=2e-3)


def test_absorb_f16(ext):
    g = torch.Generator().manual_seed(14)
    B, Sq = 16, 1
    q_raw = torch.randn(B * Sq, D.n_heads * D.qk_head, generator=g)
    W_uk = (torch.randn(D.n_heads, D.nope, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)).to(H16)
    got = ext.absorb(gpu(q_raw), gpu(W_uk), B, Sq, D.rope).cpu()
    assert got.dtype == H16
    ref = R.step_absorb(rh(q_raw).double(), W_uk.double(), B, Sq, D.nope, torch.float64)
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("B,Sq,Sk,causal", [(2, 1, 4989, False), (1, 8, 300, True)])
def test_attention_steps_f16(ext, B, Sq, Sk, causal):
    g = torch.Generator().manual_seed(Sk + 1)
    mk = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(H16)  # noqa: E731
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
    w = rh(p.cpu()[:, :Sk] * a).double().reshape(B, Sq * D.n_heads, Sk)
    rctx = torch.bmm(w, ck.double()).reshape(B, Sq, D.n_heads, -1).float()
    torch.testing.assert_close(ctx.cpu(), rctx, rtol=1e-4, atol=1e-3)
    out = ext.out(ctx, rs, gpu(wuv)).cpu()
    assert out.dtype == H16
    cn = rh(ctx.cpu() / rs.cpu().reshape(B, Sq, D.n_heads, 1))
    rout = torch.einsum("bshr,hdr->bshd", cn.double(), wuv.double()).float()
    torch.testing.assert_close(out.float(), rout, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("path", ["fused", "split"])
@pytest.mark.parametrize("Sk", [64, 16384])
def test_attention_f16_like_check_dtypes(ext, monkeypatch, path, Sk):
    """check_dtypes.py's float16 rows: B = Sq = 1, randn inputs, the output in float16 and
    its error relative to the float64 reference's largest element below 3e-2."""
    if path == "split":
        monkeypatch.setenv("MLA_ATTENTION_PATH", "split")
    else:
        monkeypatch.delenv("MLA_ATTENTION_PATH", raising=False)
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(H16)  # noqa: E731
    qa, qr = mk(1, 1, D.n_heads, D.kv_rank), mk(1, 1, D.n_heads, D.rope)
    ck, pe = mk(1, Sk, D.kv_rank), mk(1, Sk, D.rope)
    wuv = mk(D.n_heads, D.v, D.kv_rank)
    out = ext.mla_attention(*(gpu(t) for t in (qa, qr, ck, pe, wuv)), SCALE).cpu()
    assert out.dtype == H16
    ref = R.mla_attention_official(qa.double(), qr.double(), ck.double(), pe.double(),
                                   wuv.double(), SCALE)
    rel = ((out.double() - ref).abs().max() / ref.abs().max()).item()
    print(f"fp16 {path} Sk={Sk}: max rel {rel:.2e}", flush=True)
    assert rel < 3e-2


def run_layer(ext, inp, causal=False):
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], D.nope)
    g = {k: gpu(v) for k, v in inp.items()}
    qa, qr = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"],
                            gpu(W_uk.contiguous()), g["positions"], D.nope, D.rope, 1e-6)
    out = ext.mla_attention(qa, qr, g["c_kv"], g["pe_cache"], gpu(W_uv.contiguous()), SCALE,
                            causal)
    return qa, qr, out


def layer_ref(inp, causal=False):
    f32 = {k: (v.float() if v.is_floating_point() else v) for k, v in inp.items()}
    return R.mla_layer(f32["x"], f32["W_q_a"], f32["q_norm_w"], f32["W_q_b"], f32["wkv_b"],
                       f32["c_kv"], f32["pe_cache"], f32["positions"], causal=causal)


@pytest.mark.parametrize("B,Sq,Sk,causal", [(4, 1, 4989, False), (1, 1, 512, False),
                                            (2, 3, 1000, False), (1, 8, 700, True)])
def test_layer_f16_vs_fp32_oracle(ext, B, Sq, Sk, causal):
    inp = R.make_inputs(B, Sq, Sk, seed=1, dtype=H16)
    qa, qr, out = run_layer(ext, inp, causal)
    assert out.dtype == H16 and qa.dtype == H16 and qr.dtype == H16
    torch.testing.assert_close(out.float().cpu(), layer_ref(inp, causal), rtol=1e-2, atol=1e-2)


def test_layer_f16_b128_full_size(ext):
    """fp16 decode at the bf16 configuration's size (B=128, Sq=1, Sk=4989); every
    sequence against the fp32 oracle on the fp16-rounded inputs."""
    inp = R.make_inputs(128, 1, 4989, seed=0, dtype=H16)
    qa, qr, out = run_layer(ext, inp)
    assert torch.isfinite(out.float()).all()
    torch.testing.assert_close(out.float().cpu(), layer_ref(inp), rtol=1e-2, atol=1e-2)


def test_f16_restart_on_growing_scores(ext):
    """fp16 rounds P^T to a format that stops at 65504, so its reference headroom is 2^15:
    a row whose scores climb by 40 log2 units over the keys raises its reference (and
    repeats the pass) several times; the result must still match the oracle."""
    B, Sq, Sk = 1, 1, 2048
    g = torch.Generator().manual_seed(21)
    qa = torch.zeros(B, Sq, D.n_heads, D.kv_rank)
    qa[..., 0] = 1.0
    qr = torch.zeros(B, Sq, D.n_heads, D.rope)
    ck = 0.01 * torch.randn(B, Sk, D.kv_rank, generator=g)
    # score of key k for every row: ramp from 0 to 40 log2 units (s / scale * log2 e)
    ck[..., 0] = torch.linspace(0.0, 40.0 * SCALE / math.log2(math.e), Sk)
    pe = torch.zeros(B, Sk, D.rope)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)
    t = [x.to(H16) for x in (qa, qr, ck, pe, wuv)]
    out = ext.mla_attention(*(gpu(x) for x in t), SCALE).cpu()
    assert torch.isfinite(out.float()).all()
    ref = R.mla_attention_official(*(x.double() for x in t), SCALE)
    torch.testing.assert_close(out.double(), ref, rtol=2e-2, atol=2e-2)
