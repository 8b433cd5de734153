"""GPU parity of the fused attention (3a+3b+3c in one pass over the cache, flash.hip).

mla_attention takes the fused path for bf16 and fp32 at R = 512, D = 64;
MLA_ATTENTION_PATH=split selects the per-step kernels.  Both are held to the float64
oracle on the very values the kernels read, and to each other.  The queries have the
layer's spread (scores of unit standard deviation, tests/attn_cases.py), so the softmax
is far from flat; tolerances are fp32 rtol/atol 1e-4 and bf16 rtol 2e-2 with atol 2e-3
(fp16 1e-2 / 1e-3) on the long-cache outputs of standard deviation ~0.03, an atol that
grows with the output's largest element only where a few keys make the outputs O(1)
(attn_cases.tol).  tests/test_parity_power_cpu.py shows on these inputs that a dropped
rope term, an ignored causal mask, a flat softmax, a wrong score scale or a stale key
block each fail them.  Shapes cover a partial last key block, a single key, key splits
merged across workgroups (small B), causal masks with Sq > 1, splits that a tile's causal
limit leaves empty, row tiles that do not fill 64 rows (H = 40, H = 1), and a row maximum
that keeps rising: past the bf16 kernel's rescale slack, and past the fp32 kernel's
exponent headroom (which restarts its pass).
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
F32 = torch.float32
TOLS = {F32: C.TOL_F32}
DTYPES = pytest.mark.parametrize("dt", [BF, F32], ids=["bf16", "f32"])


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


def gpu(t):
    return t.to(DEV)


def inputs(B, Sq, Sk, H=D.n_heads, seed=0, dt=BF):
    return C.attn_inputs(B, Sq, Sk, H=H, seed=seed, dt=dt)


def close(got, ref, dt):
    torch.testing.assert_close(got, ref, **C.tol(dt, ref))


def oracle(args, causal):
    qa, qr, ck, pe, wuv = (t.double() for t in args)
    return R.mla_attention_official(qa, qr, ck, pe, wuv, SCALE, causal=causal).float()


def run(ext, args, causal, path=None, monkeypatch=None):
    if path is not None:
        monkeypatch.setenv("MLA_ATTENTION_PATH", path)
    try:
        out = ext.mla_attention(*(gpu(t) for t in args), SCALE, causal)
        torch.cuda.synchronize()
    finally:
        if path is not None:
            monkeypatch.delenv("MLA_ATTENTION_PATH")
    assert out.dtype == args[0].dtype
    return out.float().cpu()


SHAPES = C.FUSED_CASES


@DTYPES
@pytest.mark.parametrize("B,Sq,Sk,causal", SHAPES)
def test_fused_vs_oracle(ext, dt, B, Sq, Sk, causal):
    args = inputs(B, Sq, Sk, seed=Sk + B, dt=dt)
    close(run(ext, args, causal), oracle(args, causal), dt)


@DTYPES
@pytest.mark.parametrize("B,Sq,Sk,causal", SHAPES[2:7])
def test_fused_vs_split_path(ext, monkeypatch, dt, B, Sq, Sk, causal):
    args = inputs(B, Sq, Sk, seed=7 * Sk + B, dt=dt)
    fused = run(ext, args, causal)
    split = run(ext, args, causal, "split", monkeypatch)
    close(fused, split, dt)


@DTYPES
@pytest.mark.parametrize("B,Sq,Sk,H,causal", [(2, 3, 257, 40, False), (1, 512, 1024, 1, True),
                                              (3, 1, 100, 1, False)])
def test_fused_partial_row_tiles(ext, dt, B, Sq, Sk, H, causal):
    args = inputs(B, Sq, Sk, H=H, seed=H + Sk, dt=dt)
    close(run(ext, args, causal), oracle(args, causal), dt)


def test_fused_rising_row_max(ext):
    """Scores grow along the keys by ~0.35 (log2 units) per key, so every 32-key block
    raises the row maximum by more than the kernel's slack and rescales its state."""
    B, Sq, Sk = 2, 1, 640
    qa, qr, ck, pe, wuv = inputs(B, Sq, Sk, seed=11)
    u = torch.randn(D.kv_rank, generator=torch.Generator().manual_seed(12))
    u = u / u.norm()
    qa = (u * 64.0).expand(B, Sq, D.n_heads, D.kv_rank).to(BF)
    # s_k = 64 * 0.0525 k = 3.36 k, i.e. t_k = s_k / sqrt(192) * log2(e) = 0.35 k; the
    # keys stay O(10), so the bf16 rounding of p stays within the tolerance
    ramp = torch.arange(Sk, dtype=torch.float32) * 0.0525
    ck = (ck.float() * 0.05 + ramp[None, :, None] * u).to(BF)
    args = (qa, qr, ck, pe, wuv)
    close(run(ext, args, False), oracle(args, False), BF)


# bf16 and fp16 run on two kernels: eight specialised waves (flash16x_kernel, the default:
# score waves, and P.V waves one key block behind that share each row's reference; the P.V
# waves over 64 rows x 128 columns, or 32 x 256 with MLA_FLASH16_PV=32) or four key-split
# waves (flash16_kernel, MLA_FLASH16_SPEC=0); every variant must match the oracle everywhere
H16 = torch.float16
FP16_KERNELS = pytest.mark.parametrize("spec", ["1", "pv32", "0"],
                                       ids=["specialised", "specialised-pv32", "key-split"])


def set_16bit_kernel(monkeypatch, spec):
    """specialised waves with the P.V waves over 64 rows x 128 columns (the default) or 32
    rows x 256 columns (MLA_FLASH16_PV=32), or the key-split waves (MLA_FLASH16_SPEC=0)"""
    monkeypatch.setenv("MLA_FLASH16_SPEC", "0" if spec == "0" else "1")
    if spec == "pv32":
        monkeypatch.setenv("MLA_FLASH16_PV", "32")
    else:
        monkeypatch.delenv("MLA_FLASH16_PV", raising=False)
HALF_DTYPES = pytest.mark.parametrize("dt", [BF, H16], ids=["bf16", "f16"])


@FP16_KERNELS
@HALF_DTYPES
@pytest.mark.parametrize("B,Sq,Sk,H,causal", C.FLASH16_CASES)
def test_16bit_kernels_vs_oracle(ext, monkeypatch, spec, dt, B, Sq, Sk, H, causal):
    set_16bit_kernel(monkeypatch, spec)
    args = inputs(B, Sq, Sk, H=H, seed=3 * Sk + B, dt=dt)
    close(run(ext, args, causal), oracle(args, causal), dt)


@FP16_KERNELS
def test_16bit_kernels_full_size(ext, monkeypatch, spec):
    """B=128, Sk=4989 in bf16 (the cfg4 attention) on either 16-bit kernel, every sequence
    against the oracle."""
    set_16bit_kernel(monkeypatch, spec)
    args = inputs(128, 1, 4989, seed=78, dt=BF)
    ref = R.mla_attention_official(*(t.float() for t in args), SCALE)
    close(run(ext, args, False), ref, BF)


@pytest.mark.parametrize("kind", ["bf16", "f16", "fp8-code-ring", "fp8-convert"])
def test_normalised_16bit_ctx_same_bits(ext, monkeypatch, kind):
    """With one key split (B = 128) the default 16-bit passes write ctx already divided by
    its row sum and rounded to the storage format -- the values 3d's staging forms from the
    fp32 ctx and row sum -- so the output equals the MLA_CTX16=0 path bit for bit; and it
    matches the oracle."""
    def call():
        if kind.startswith("fp8"):
            return ext.mla_attention_fp8kv(*(gpu(t) for t in f8[:4]), f8[4], gpu(f8[5]),
                                           SCALE).cpu()
        return ext.mla_attention(*(gpu(t) for t in args), SCALE).cpu()

    if kind.startswith("fp8"):
        if kind == "fp8-convert":
            monkeypatch.setenv("MLA_FLASH16_FP8", "convert")
        f8 = C.fp8_inputs(128, 1, 1000, seed=9)
        ref = R.mla_attention_fp8kv(*f8, SCALE)
        dt = BF
    else:
        dt = BF if kind == "bf16" else H16
        args = inputs(128, 1, 1000, seed=9, dt=dt)
        ref = oracle(args, False)
    out16 = call()
    monkeypatch.setenv("MLA_CTX16", "0")
    out32 = call()
    assert torch.equal(out16, out32)
    close(out16.float(), ref.float(), dt)


@FP16_KERNELS
@HALF_DTYPES
def test_16bit_kernels_repeat_passes(ext, monkeypatch, spec, dt):
    """Every row's scores climb along the keys past the kernel's headroom over its reference
    (2^15 for fp16, 2^64 for bf16) several times: each pass raises the references and the
    pass repeats with them (in the specialised kernel both key halves of a row must agree on
    the raised reference before they add into one O)."""
    set_16bit_kernel(monkeypatch, spec)
    B, Sq, Sk = 2, 1, 2048
    climb = 40.0 if dt == H16 else 200.0        # log2 units from the first key to the last
    g = torch.Generator().manual_seed(23)
    qa = torch.zeros(B, Sq, D.n_heads, D.kv_rank)
    qa[..., 0] = 1.0
    qr = torch.zeros(B, Sq, D.n_heads, D.rope)
    ck = 0.01 * torch.randn(B, Sk, D.kv_rank, generator=g)
    ck[..., 0] = torch.linspace(0.0, climb * SCALE / math.log2(math.e), Sk)
    pe = torch.zeros(B, Sk, D.rope)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)
    args = tuple(x.to(dt) for x in (qa, qr, ck, pe, wuv))
    out = run(ext, args, False)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out, oracle(args, False), rtol=2e-2, atol=2e-2)


# fp32 runs on three kernels: 64-row workgroups when the batch fills the chip, on eight
# specialised waves (flash32x_kernel, the default) or four (flash32_kernel,
# MLA_FLASH32_SPEC=0), and 16-row workgroups of key-split waves (flash32w_kernel) when it
# would need key splits; MLA_FLASH32_WAVE=0 / 1 forces the 64-row or the 16-row kind, and
# every kernel must match the oracle everywhere
FP32_KERNELS = pytest.mark.parametrize("wave", ["0", "0s", "1"], ids=["wg64-spec", "wg64", "wave16"])


def set_fp32_kernel(monkeypatch, wave):
    monkeypatch.setenv("MLA_FLASH32_WAVE", wave[0])
    monkeypatch.setenv("MLA_FLASH32_SPEC", "0" if wave == "0s" else "1")


@FP32_KERNELS
@pytest.mark.parametrize("B,Sq,Sk,H,causal", [
    (1, 1, 1, 128, False), (1, 1, 17, 128, False), (1, 1, 4989, 128, False),
    (8, 1, 4989, 128, False), (3, 2, 300, 128, True), (2, 16, 1000, 128, True),
    (2, 3, 257, 40, False), (1, 512, 1024, 1, True), (40, 1, 700, 128, False),
    (1, 1, 65, 128, False)])
def test_fp32_kernels_vs_oracle(ext, monkeypatch, wave, B, Sq, Sk, H, causal):
    set_fp32_kernel(monkeypatch, wave)
    args = inputs(B, Sq, Sk, H=H, seed=3 * Sk + B, dt=F32)
    close(run(ext, args, causal), oracle(args, causal), F32)


@FP32_KERNELS
def test_fp32_kernels_full_size(ext, monkeypatch, wave):
    """B=128, Sk=4989 on either kernel (the key-split waves at a full grid: no key split,
    1,024 workgroups), every sequence against the oracle."""
    set_fp32_kernel(monkeypatch, wave)
    args = inputs(128, 1, 4989, seed=77, dt=F32)
    got = run(ext, args, False)
    qa, qr, ck, pe, wuv = args
    ref = R.mla_attention_official(qa, qr, ck, pe, wuv, SCALE)
    torch.testing.assert_close(got, ref, **TOLS[F32])


@pytest.mark.parametrize("small", ["1", "0"], ids=["fused-3d", "gemm-3d"])
@pytest.mark.parametrize("B,Sq,Sk,causal", [(1, 1, 4989, False), (3, 1, 4989, False),
                                            (3, 1, 100, False), (1, 4, 700, True),
                                            (1, 4, 64, True), (1, 1, 33, False),
                                            (4, 1, 512, False), (4, 1, 4989, False),
                                            (8, 1, 4989, False), (5, 1, 1000, False),
                                            (2, 4, 700, True), (1, 8, 64, True),
                                            (8, 1, 64, False)])
def test_fp32_decode_3d_with_merge(ext, monkeypatch, small, B, Sq, Sk, causal):
    """At B*Sq <= 4 (fp32) with at most 128 split rows per head to merge, mla_attention runs
    3d on a kernel that also merges the pass's key splits, and at B*Sq <= 8 on the same
    kernel reading ctx / row_sum, written by the pass when it ran unsplit (Sk = 64) or else
    by the merge kernel (B*Sq = 5..8 split); MLA_OUT_SMALL=0 keeps the merge kernel and the
    3d GEMM.  Both against the oracle."""
    monkeypatch.setenv("MLA_OUT_SMALL", small)
    args = inputs(B, Sq, Sk, seed=5 * Sk + B, dt=F32)
    close(run(ext, args, causal), oracle(args, causal), F32)


@DTYPES
@pytest.mark.parametrize("B,Sq,Sk", [(132, 1, 4989), (200, 1, 1000), (70, 4, 700)])
def test_fused_key_split_past_one_round(ext, dt, B, Sq, Sk):
    """Batches just past one workgroup per CU (264, 400 and 560 workgroups per split): the
    planner splits the keys so that the last round is not nearly empty; every sequence
    against the oracle."""
    args = inputs(B, Sq, Sk, seed=B + Sk, dt=dt)
    close(run(ext, args, False), oracle(args, False), dt)


@FP32_KERNELS
@pytest.mark.parametrize("jump", [100.0, 400.0])
def test_fused_f32_restart(ext, monkeypatch, wave, jump):
    """fp32 keeps each row's exponentials against the first visible block's maximum; a
    row whose later maximum passes it by the 2^64 headroom restarts the pass.  Here the
    scores rise by `jump` (log2 units) over the keys in steps of ~0.35 per key, so the
    kernel restarts one (100) or several (400) times; a one-key spike at key 900 of
    another sequence restarts from a late block."""
    set_fp32_kernel(monkeypatch, wave)
    B, Sq, Sk = 2, 1, 1200
    qa, qr, ck, pe, wuv = inputs(B, Sq, Sk, seed=13, dt=F32)
    u = torch.randn(D.kv_rank, generator=torch.Generator().manual_seed(14))
    u = u / u.norm()
    qa = (u * 64.0).expand(B, Sq, D.n_heads, D.kv_rank).contiguous()
    # t_k = s_k / sqrt(192) * log2(e); s_k = 64 * a * k with a chosen so t_(Sk-1) = jump
    a = jump / (Sk - 1) * SCALE / math.log2(math.e) / 64.0
    ramp = torch.arange(Sk, dtype=torch.float32) * a
    ck = ck * 0.05
    ck[0] += ramp[:, None] * u
    ck[1, 900] += (jump / math.log2(math.e) * SCALE / 64.0) * u
    args = (qa, qr, ck, pe, wuv)
    torch.testing.assert_close(run(ext, args, False), oracle(args, False), **TOLS[F32])


@DTYPES
def test_fused_deterministic(ext, dt):
    args = [gpu(t) for t in inputs(3, 1, 2000, seed=5, dt=dt)]
    a = ext.mla_attention(*args, SCALE)
    b = ext.mla_attention(*args, SCALE)
    assert torch.equal(a, b)


@DTYPES
def test_fused_full_size_vs_split_path(ext, monkeypatch, dt):
    """B=128, Sq=1, Sk=4989 (the cfg2 / cfg4 attention): the fused and per-step paths agree
    on every sequence; the oracle checks three of them."""
    args = inputs(128, 1, 4989, seed=0, dt=dt)
    fused = run(ext, args, False)
    split = run(ext, args, False, "split", monkeypatch)
    close(fused, split, dt)
    pick = [0, 77, 127]
    ref = oracle(tuple(t[pick] for t in args[:4]) + (args[4],), False)
    close(fused[pick], ref, dt)


@DTYPES
@pytest.mark.parametrize("B,Sq,Sk,causal", [(2, 1, 300, False), (1, 1, 4989, False),
                                            (2, 4, 500, True)])
def test_attn_ctx_step_vs_oracle(ext, monkeypatch, dt, B, Sq, Sk, causal):
    """The per-step fused entry point: ctx / row_sum equals the oracle's softmax-weighted
    c_kv (float64 reference on the values the kernel reads; bf16 P is rounded only in the
    kernel), and feeding (ctx, row_sum) to the 3d step gives mla_attention's output bit
    for bit when mla_attention runs the same 3d GEMM (decode-sized fp32 batches otherwise
    take 3d with the split merge folded in, equal to rounding)."""
    qa, qr, ck, pe, wuv = inputs(B, Sq, Sk, seed=3 * Sk + B, dt=dt)
    ctx, rs = ext.attn_ctx(gpu(qa), gpu(qr), gpu(ck), gpu(pe), SCALE, causal)
    assert ctx.dtype == torch.float32 and ctx.shape == (B, Sq, D.n_heads, D.kv_rank)
    assert rs.shape == (B * Sq * D.n_heads,) and bool((rs > 0).all())
    got = (ctx / rs.reshape(B, Sq, D.n_heads, 1)).cpu()
    s = (torch.einsum("bqhr,bkr->bqhk", qa.double(), ck.double())
         + torch.einsum("bqhd,bkd->bqhk", qr.double(), pe.double())) / SCALE
    if causal:
        s = s.masked_fill(~R.causal_mask(Sq, Sk)[None, :, None, :], float("-inf"))
    ref = torch.einsum("bqhk,bkr->bqhr", torch.softmax(s, dim=-1), ck.double()).float()
    close(got, ref, dt)
    out = ext.out(ctx, rs, gpu(wuv))
    own = ext.mla_attention(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(wuv), SCALE, causal)
    monkeypatch.setenv("MLA_OUT_SMALL", "0")
    full = ext.mla_attention(gpu(qa), gpu(qr), gpu(ck), gpu(pe), gpu(wuv), SCALE, causal)
    assert torch.equal(out, full)
    close(own.float().cpu(), full.float().cpu(), dt)


@pytest.mark.parametrize("B,Sq,Sk,causal", [(40, 1, 700, False), (2, 16, 1000, True),
                                            (130, 1, 333, False)])
def test_fp32_specialised_waves_same_bits(ext, monkeypatch, B, Sq, Sk, causal):
    """The eight specialised waves (flash32x_kernel, whose P.V waves change their wave
    priority within each step) run the four-wave kernel's MFMAs in the same order on the same
    P values: the output is the same bit for bit."""
    monkeypatch.setenv("MLA_FLASH32_WAVE", "0")
    args = inputs(B, Sq, Sk, seed=7 * Sk + B, dt=F32)
    monkeypatch.setenv("MLA_FLASH32_SPEC", "1")
    spec = run(ext, args, causal)
    monkeypatch.setenv("MLA_FLASH32_SPEC", "0")
    four = run(ext, args, causal)
    assert torch.equal(spec, four)


@pytest.mark.parametrize("B,Sq,Sk,causal", [(8, 1, 4989, False), (3, 4, 700, True)])
def test_bf16_pv_layouts_same_bits(ext, monkeypatch, B, Sq, Sk, causal):
    """The default 16-bit pass (P.V waves over 64 rows x 128 columns, with their wave
    priority raised for the first MFMAs of each step) and the 32 x 256 layout
    (MLA_FLASH16_PV=32) add the same products in the same order: the same bits."""
    args = inputs(B, Sq, Sk, seed=11 * Sk + B, dt=BF)
    monkeypatch.delenv("MLA_FLASH16_PV", raising=False)
    a = run(ext, args, causal)
    monkeypatch.setenv("MLA_FLASH16_PV", "32")
    b = run(ext, args, causal)
    assert torch.equal(a, b)
