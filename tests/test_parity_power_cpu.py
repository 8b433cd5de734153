"""The attention parity tests can fail: on each GPU test's own inputs (same builders, shapes
and seeds, from tests/attn_cases.py), an oracle with one planted mistake -- the rope term
dropped, the causal mask ignored, a flat softmax, scores off by 4x, P.V reading the previous
key block's rows, the fp8 scale applied twice -- lands outside that test's tolerance, while
the oracle with the kernel's own 16-bit roundings stays inside it.  CPU only: the mistakes
are planted in the oracle, never in a kernel.

A mistake that the case cannot show (any score mistake with one visible key, a stale block
with at most 32 keys, the causal mask on a non-causal case) leaves the output unchanged;
those pairs are checked to be equal instead.
"""

from __future__ import annotations

import pytest
import torch

import attn_cases as C
from oracle import mla_ref as R

D = C.D


def observable(mistake, max_keys, causal):
    if mistake == "no_causal":
        return causal
    if mistake == "stale_v":
        return max_keys > 32
    return max_keys > 1


def check_power(ref, variant, mistakes, tol, max_keys, causal):
    """Every observable mistake violates tol against ref; every other one leaves the
    (float64) variant without a mistake unchanged."""
    base = variant(None)
    assert not C.violates(base, ref, rtol=1e-4, atol=1e-6)
    for m in mistakes:
        got = variant(m)
        if observable(m, max_keys, causal):
            assert C.violates(got, ref, **tol), f"mistake {m!r} passes the tolerance {tol}"
        else:
            torch.testing.assert_close(got, base, rtol=1e-9, atol=1e-12)


def round_like_kernel(qa, qr, ck, pe, wuv, causal, dt):
    """The attention with the roundings a 16-bit kernel makes: P (against the row maximum)
    rounded to dt before P.V, ctx / row_sum rounded to dt before 3d, and the output stored
    in dt.  Used to show the tolerance leaves room for a correct kernel."""
    qa, qr, ck, pe, wuv = (t.double() for t in (qa, qr, ck, pe, wuv))
    B, Sq, H, Rk = qa.shape
    Sk = ck.shape[1]
    s = (torch.bmm(qa.reshape(B, Sq * H, Rk), ck.transpose(1, 2).contiguous())
         + torch.bmm(qr.reshape(B, Sq * H, -1), pe.transpose(1, 2).contiguous())) / C.SCALE
    if causal:
        vis = R.causal_mask(Sq, Sk).repeat_interleave(H, dim=0)
        s = s.masked_fill(~vis.unsqueeze(0), float("-inf"))
    p = torch.exp(s - s.amax(dim=-1, keepdim=True))
    l = p.sum(dim=-1, keepdim=True)
    ctx = torch.bmm(p.to(dt).double(), ck) / l
    out = torch.einsum("bshr,hdr->bshd", ctx.to(dt).double().reshape(B, Sq, H, Rk), wuv)
    return out.to(dt).double()


# ---- the claim about the inputs' spread

def test_layer_queries_have_the_layers_spread():
    """The real Q path (oracle.mla_ref.prepare_q_mla_absorbed on make_inputs' seeded
    weights) gives q_absorbed with std ~0.5, q_rope with std ~1 and scores against a N(0,1)
    cache with std ~1 -- the statistics attn_cases.layer_queries draws from."""
    inp = R.make_inputs(8, 1, 256, seed=3)
    W_uk, _ = R.split_wkv_b(inp["wkv_b"], D.nope)
    qa, qr = R.prepare_q_mla_absorbed(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                      W_uk, inp["positions"], D.nope, D.rope)
    assert abs(qa.std().item() / C.LAYER_QA_STD - 1) < 0.1
    assert abs(qr.std().item() / C.LAYER_QR_STD - 1) < 0.1
    s = (torch.einsum("bqhr,bkr->bqhk", qa, inp["c_kv"])
         + torch.einsum("bqhd,bkd->bqhk", qr, inp["pe_cache"])) / C.SCALE
    assert 0.85 < s.std().item() < 1.15
    g = torch.Generator().manual_seed(0)
    qa2, qr2 = C.layer_queries(g, 8, 1)
    s2 = (torch.einsum("bqhr,bkr->bqhk", qa2, inp["c_kv"])
          + torch.einsum("bqhd,bkd->bqhk", qr2, inp["pe_cache"])) / C.SCALE
    assert 0.9 < s2.std().item() / s.std().item() < 1.1


def test_variant_without_mistake_is_the_oracle():
    args = C.attn_inputs(2, 3, 100, seed=1, dt=torch.float32)
    for causal in (False, True):
        ref = R.mla_attention_official(*args, C.SCALE, causal=causal)
        torch.testing.assert_close(C.attention(*args, causal=causal).float(), ref,
                                   rtol=1e-5, atol=1e-6)


# ---- fp8 cache (tests/test_gpu_fp8kv.py)

@pytest.mark.parametrize("B,Sq,Sk,causal", C.FP8_DENSE_CASES)
def test_fp8_dense_cases_reject_mistakes(B, Sq, Sk, causal):
    qa, qr, ck, pe, ks, wuv = C.fp8_inputs(B, Sq, Sk, seed=B * 100 + Sk)
    ref = R.mla_attention_fp8kv(qa, qr, ck, pe, ks, wuv, C.SCALE, causal)
    check_power(ref, lambda m: C.fp8_attention(qa, qr, ck, pe, ks, wuv, causal, m),
                C.MISTAKES_FP8, C.tol(C.BF, ref), Sk, causal)
    dec = (R.decode_e4m3(ck, ks), R.decode_e4m3(pe, ks))
    near = round_like_kernel(qa, qr, *dec, wuv, causal, C.BF)
    assert not C.violates(near, ref, **C.tol(C.BF, ref))


def test_fp8_full_size_case_rejects_mistakes():
    """The B=128, Sk=4989 case; the first four sequences suffice (assert_close over all of
    them fails wherever any one fails)."""
    qa, qr, ck, pe, ks, wuv = C.fp8_inputs(128, 1, 4989, seed=C.FP8_FULL_SEED)
    sub = slice(0, 4)
    qa, qr, ck, pe = qa[sub], qr[sub], ck[sub], pe[sub]
    ref = R.mla_attention_fp8kv(qa, qr, ck, pe, ks, wuv, C.SCALE)
    check_power(ref, lambda m: C.fp8_attention(qa, qr, ck, pe, ks, wuv, False, m),
                C.MISTAKES_FP8, C.tol(C.BF, ref), 4989, False)


@pytest.mark.parametrize("page,lens,causal,Sq", C.FP8_PAGED_CASES)
def test_fp8_paged_cases_reject_mistakes(page, lens, causal, Sq):
    B = len(lens)
    max_pages = max(1, -(-max(lens) // page))
    qa, qr, ck, pe, table, sl, ks, wuv = C.paged_fp8_inputs(B, Sq, lens, page, max_pages,
                                                            seed=page + 7 * B)
    ref = R.mla_attention_paged(qa.float(), qr.float(), R.decode_e4m3(ck, ks),
                                R.decode_e4m3(pe, ks), table, sl, wuv.float(), C.SCALE, causal)
    check_power(ref, lambda m: C.paged_fp8_attention(qa, qr, ck, pe, table, sl, ks, wuv,
                                                     causal, m),
                C.MISTAKES_FP8, C.tol(C.BF, ref), max(lens), causal)


def test_fp8_paged_full_size_case_rejects_mistakes():
    lens = C.fp8_full_paged_lens()
    qa, qr, ck, pe, table, sl, ks, wuv = C.paged_fp8_inputs(128, 1, lens, 64, -(-4989 // 64),
                                                            seed=128)
    sub = slice(0, 4)     # lens[0] = 4989 and lens[1] = 1 are among them
    qa, qr, table, sl = qa[sub], qr[sub], table[sub], sl[sub]
    ref = R.mla_attention_paged(qa.float(), qr.float(), R.decode_e4m3(ck, ks),
                                R.decode_e4m3(pe, ks), table, sl, wuv.float(), C.SCALE)
    check_power(ref, lambda m: C.paged_fp8_attention(qa, qr, ck, pe, table, sl, ks, wuv,
                                                     False, m),
                C.MISTAKES_FP8, C.tol(C.BF, ref), 4989, False)


# ---- 16-bit and fp32 fused kernels (tests/test_gpu_flash.py)

HALF = pytest.mark.parametrize("dt", [C.BF, C.H16], ids=["bf16", "f16"])


def flash_ref(args, causal):
    """test_gpu_flash's oracle: float64 on the values the kernel reads."""
    return R.mla_attention_official(*(t.double() for t in args), C.SCALE,
                                    causal=causal).float()


@HALF
@pytest.mark.parametrize("B,Sq,Sk,H,causal", C.FLASH16_CASES)
def test_flash16_cases_reject_mistakes(dt, B, Sq, Sk, H, causal):
    args = C.attn_inputs(B, Sq, Sk, H=H, seed=3 * Sk + B, dt=dt)
    ref = flash_ref(args, causal)
    tol = C.tol(dt, ref)
    check_power(ref, lambda m: C.attention(*args, causal=causal, mistake=m), C.MISTAKES, tol,
                Sk, causal)
    assert not C.violates(round_like_kernel(*args, causal, dt), ref, **tol)


@pytest.mark.parametrize("dt", [C.BF, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("B,Sq,Sk,causal", C.FUSED_CASES)
def test_fused_cases_reject_mistakes(dt, B, Sq, Sk, causal):
    args = C.attn_inputs(B, Sq, Sk, seed=Sk + B, dt=dt)
    ref = flash_ref(args, causal)
    tol = C.tol(dt, ref)
    check_power(ref, lambda m: C.attention(*args, causal=causal, mistake=m), C.MISTAKES, tol,
                Sk, causal)
    if dt == C.BF:
        assert not C.violates(round_like_kernel(*args, causal, dt), ref, **tol)


def test_violates_matches_assert_close():
    a = torch.tensor([1.0, 2.0])
    for b in (torch.tensor([1.0, 2.03]), torch.tensor([1.0, 2.05])):
        tol = C.tol(C.BF, b)
        try:
            torch.testing.assert_close(a, b, **tol)
            closes = True
        except AssertionError:
            closes = False
        assert C.violates(a, b, **tol) == (not closes)


def test_causal_query_blocks_equal_the_full_causal_problem():
    """The cfg5 GPU test checks its 512 rows in blocks: queries s0 .. s0+n-1 of a causal
    Sq x Sk problem over keys [0, Sk - Sq + s0 + n) are the causal problem
    causal_mask(n, Sk - Sq + s0 + n).  Here, on a small shape, block by block against the
    whole."""
    B, Sq, Sk, n = 2, 12, 50, 4
    args = C.attn_inputs(B, Sq, Sk, H=3, seed=8, dt=torch.float64)
    qa, qr, ck, pe, wuv = args
    full = R.mla_attention_official(*args, C.SCALE, causal=True)
    for s0 in range(0, Sq, n):
        lim = Sk - Sq + s0 + n
        blk = R.mla_attention_official(qa[:, s0:s0 + n], qr[:, s0:s0 + n], ck[:, :lim],
                                       pe[:, :lim], wuv, C.SCALE, causal=True)
        torch.testing.assert_close(blk, full[:, s0:s0 + n], rtol=1e-12, atol=1e-12)
