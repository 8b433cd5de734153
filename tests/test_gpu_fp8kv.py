"""GPU parity of attention over an fp8 KV cache (mla_attention_fp8kv,
mla_attention_paged_fp8kv).

The cache holds OCP E4M3 codes (torch.float8_e4m3fn) of value / kv_scale; queries, W_uv and
the output are bf16.  The oracle decodes the codes with its own restated E4M3 table
(oracle/mla_ref.py e4m3_values, pinned against torch's float8_e4m3fn in test_oracle.py) and
runs the attention in float32.  The queries have the layer's spread (scores with unit
standard deviation, tests/attn_cases.py), and the tolerance is rtol 2e-2 with atol 2e-3 on
outputs of standard deviation ~0.03 (larger only where a few keys make the outputs O(1));
tests/test_parity_power_cpu.py shows, on these very inputs, that a dropped rope term, an
ignored causal mask, a flat softmax, a wrong score scale, a stale key block or a doubled
kv_scale each fail it.  The decoder the kernel uses is checked on its own over all 256
codes.  The fused pass runs on the specialised waves with only the e4m3 codes in LDS, converted to
bf16 in registers as each fragment is read (the default), on the same waves converting each
block into a bf16 ring (MLA_FLASH16_FP8=convert), or on the key-split waves
(MLA_FLASH16_SPEC=0); the parity tests run all three.
"""

from __future__ import annotations

import pytest
import torch

import attn_cases as C
from oracle import mla_ref as R

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = R.DSV3
SCALE = C.SCALE
BF = torch.bfloat16


def check(out, ref):
    assert out.dtype == BF and torch.isfinite(out.float()).all()
    torch.testing.assert_close(out.float(), ref.float(), **C.tol(BF, ref))


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


@pytest.mark.parametrize("scale", [1.0, 0.375])
def test_fp8_decoder_all_codes(ext, scale):
    """The kernel's e4m3 -> bf16 -> fp32 decoding of every code equals the format's value
    (NaN exactly at 0x7F and 0xFF), times the scale."""
    codes = torch.arange(256, dtype=torch.uint8)
    got = ext.fp8_dequantize(codes.to(DEV), scale).cpu()
    want = R.e4m3_values() * scale
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan], want[~nan])
    # odd lengths take the tail path of the decoder
    got7 = ext.fp8_dequantize(codes[:7].to(DEV), scale).cpu()
    assert torch.equal(got7, want[:7])


fp8_inputs = C.fp8_inputs


# the fp8 pass on the specialised waves with only the codes in LDS (the default), the same
# waves converting each block into a bf16 ring (MLA_FLASH16_FP8=convert), or the key-split
# waves (MLA_FLASH16_SPEC=0)
KERNELS = pytest.mark.parametrize("spec", ["1", "convert", "0"],
                                  ids=["code-ring", "convert-ring", "key-split"])


def set_fp8_kernel(monkeypatch, spec):
    monkeypatch.setenv("MLA_FLASH16_SPEC", "0" if spec == "0" else "1")
    if spec == "convert":
        monkeypatch.setenv("MLA_FLASH16_FP8", "convert")
    else:
        monkeypatch.delenv("MLA_FLASH16_FP8", raising=False)


@KERNELS
@pytest.mark.parametrize("B,Sq,Sk,causal", C.FP8_DENSE_CASES)
def test_fp8kv_attention_matches_oracle(ext, monkeypatch, spec, B, Sq, Sk, causal):
    set_fp8_kernel(monkeypatch, spec)
    qa, qr, ck, pe, kv_scale, wuv = fp8_inputs(B, Sq, Sk, seed=B * 100 + Sk)
    out = ext.mla_attention_fp8kv(*(t.to(DEV) for t in (qa, qr, ck, pe)), kv_scale, wuv.to(DEV),
                                  SCALE, causal).cpu()
    check(out, R.mla_attention_fp8kv(qa, qr, ck, pe, kv_scale, wuv, SCALE, causal))


def test_fp8kv_uint8_codes_and_scale(ext):
    """The cache may come as raw uint8 codes; the same codes under two scales give the
    attention of the two decoded caches."""
    qa, qr, ck, pe, kv_scale, wuv = fp8_inputs(2, 1, 777, seed=5)
    args = [t.to(DEV) for t in (qa, qr)]
    for s in (kv_scale, 2.5 * kv_scale):
        out = ext.mla_attention_fp8kv(*args, ck.view(torch.uint8).to(DEV),
                                      pe.view(torch.uint8).to(DEV), s, wuv.to(DEV), SCALE).cpu()
        check(out, R.mla_attention_fp8kv(qa, qr, ck, pe, s, wuv, SCALE))


@KERNELS
def test_fp8kv_b128_full_size(ext, monkeypatch, spec):
    """B=128 decode at Sk=4989 (the bf16 configuration's shape) over an fp8 cache, every
    sequence against the oracle."""
    set_fp8_kernel(monkeypatch, spec)
    qa, qr, ck, pe, kv_scale, wuv = fp8_inputs(128, 1, 4989, seed=C.FP8_FULL_SEED)
    out = ext.mla_attention_fp8kv(*(t.to(DEV) for t in (qa, qr, ck, pe)), kv_scale, wuv.to(DEV),
                                  SCALE).cpu()
    check(out, R.mla_attention_fp8kv(qa, qr, ck, pe, kv_scale, wuv, SCALE))


def test_fp8kv_close_to_the_bf16_cache(ext):
    """Against the bf16 path on the same (decoded) cache values the two kernels agree to
    the bf16 tolerance."""
    qa, qr, ck, pe, kv_scale, wuv = fp8_inputs(2, 1, 3000, seed=11)
    out8 = ext.mla_attention_fp8kv(*(t.to(DEV) for t in (qa, qr, ck, pe)), kv_scale,
                                   wuv.to(DEV), SCALE).cpu().float()
    ck16 = (ck.float() * kv_scale).to(BF)
    pe16 = (pe.float() * kv_scale).to(BF)
    out16 = ext.mla_attention(*(t.to(DEV) for t in (qa, qr, ck16, pe16, wuv)), SCALE).cpu().float()
    torch.testing.assert_close(out8, out16, **C.tol(BF, out16))


# ---- paged fp8 cache (mla_attention_paged_fp8kv)

paged_fp8_inputs = C.paged_fp8_inputs


def paged_fp8_oracle(qa, qr, ck, pe, table, sl, kv_scale, wuv, causal=False):
    """The paged oracle (each sequence over its own gathered keys) on the decoded pools."""
    return R.mla_attention_paged(qa.float(), qr.float(), R.decode_e4m3(ck, kv_scale),
                                 R.decode_e4m3(pe, kv_scale), table, sl, wuv.float(), SCALE,
                                 causal)


def run_paged_fp8(ext, qa, qr, ck, pe, table, sl, kv_scale, wuv, causal=False):
    return ext.mla_attention_paged_fp8kv(*(t.to(DEV) for t in (qa, qr, ck, pe, table, sl)),
                                         kv_scale, wuv.to(DEV), SCALE, causal).cpu()


@KERNELS
@pytest.mark.parametrize("page,lens,causal,Sq", C.FP8_PAGED_CASES)
def test_paged_fp8kv_matches_oracle(ext, monkeypatch, spec, page, lens, causal, Sq):
    """Ragged lengths (not multiples of the page), shuffled pools and, in the last case,
    empty sequences, whose rows are zeros as in the oracle."""
    set_fp8_kernel(monkeypatch, spec)
    B = len(lens)
    max_pages = max(1, -(-max(lens) // page))
    inp = paged_fp8_inputs(B, Sq, lens, page, max_pages, seed=page + 7 * B)
    out = run_paged_fp8(ext, *inp, causal=causal)
    check(out, paged_fp8_oracle(*inp, causal=causal))
    for b, n in enumerate(lens):
        if n == 0:
            assert not out[b].float().any()


def test_paged_fp8kv_equals_dense_layout(ext):
    """Full lengths with the pages in sequence order hold the dense cache: the paged call
    agrees with mla_attention_fp8kv on it, and with the oracle."""
    B, Sk, page = 3, 4992, 64
    qa, qr, ck, pe, kv_scale, wuv = fp8_inputs(B, 1, Sk, seed=31)
    mp = Sk // page
    table = torch.arange(B * mp, dtype=torch.int32).reshape(B, mp)
    sl = torch.full((B,), Sk, dtype=torch.int32)
    dense = ext.mla_attention_fp8kv(*(t.to(DEV) for t in (qa, qr, ck, pe)), kv_scale,
                                    wuv.to(DEV), SCALE).cpu()
    paged = run_paged_fp8(ext, qa, qr, ck.reshape(-1, page, D.kv_rank),
                          pe.reshape(-1, page, D.rope), table, sl, kv_scale, wuv)
    torch.testing.assert_close(paged.float(), dense.float(), **C.tol(BF, dense.float()))
    check(paged, R.mla_attention_fp8kv(qa, qr, ck, pe, kv_scale, wuv, SCALE))


@KERNELS
def test_paged_fp8kv_b128_ragged_full_size(ext, monkeypatch, spec):
    """B=128 decode over a ragged paged fp8 cache up to Sk=4989 keys, every sequence
    against the oracle."""
    set_fp8_kernel(monkeypatch, spec)
    lens = C.fp8_full_paged_lens()
    page = 64
    inp = paged_fp8_inputs(128, 1, lens, page, -(-4989 // page), seed=128)
    check(run_paged_fp8(ext, *inp), paged_fp8_oracle(*inp))
