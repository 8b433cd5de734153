"""Attention test inputs with the layer's score spread, the cases the 16-bit and fp8 GPU
parity tests run, and oracle variants with planted mistakes -- TEST INFRASTRUCTURE ONLY.

Why the spread matters.  The scores are t = (q_absorbed . c_kv + q_rope . pe) / sqrt(192).
If the queries are scaled down (q * 0.05, or q / sqrt(512)), t has a standard deviation
below 0.1, the softmax is almost flat, and the output is nearly the mean of the cache
rows -- a kernel that drops the rope term, scales the scores wrongly or ignores them
altogether still lands within a 16-bit tolerance.  The inputs here follow the layer's own
statistics instead (``exhaustive_benchmark_suite.py:268-286`` with the seeded weights of
``oracle.mla_ref.make_inputs``): q_nope has unit RMS (RMSNorm output times a gain near 1,
through W_q_b ~ N(0, 1/q_lora)), so q_absorbed = q_nope @ W_uk with W_uk ~ N(0, 1/kv_rank)
has variance nope / kv_rank = 0.25, and q_rope keeps q_pe's unit variance (RoPE rotates
pairs).  Then t has unit variance: (512 * 0.25 + 64 * 1) / 192 = 1.
``tests/test_parity_power_cpu.py`` checks that claim on the real Q path and proves, case
by case, that each GPU test's tolerance rejects the planted mistakes below.

The mistakes (``attention(..., mistake=...)``), each a plausible kernel bug:
  no_rope       the q_rope . pe term dropped from the 576-deep score
  no_causal     the causal mask ignored
  uniform       the scores ignored (a flat softmax over the visible keys)
  scores_div4   the scores off by a constant factor (a wrong scale)
  stale_v       P . V reading the previous 32-key block's cache rows (a stale ring stage)
  kv_scale_twice  (fp8 cache) the dequantisation scale applied twice to the cache
"""

from __future__ import annotations

import math

import torch

from oracle import mla_ref as R

D = R.DSV3
SCALE = math.sqrt(D.qk_head)
BF = torch.bfloat16
H16 = torch.float16
F8 = torch.float8_e4m3fn

LAYER_QA_STD = math.sqrt(D.nope / D.kv_rank)   # 0.5
LAYER_QR_STD = 1.0

# Tolerances of the parity tests.  fp32 is the north star's rtol/atol 1e-4.  For 16-bit
# storage and the fp8 cache, rtol is the bf16 2e-2 (fp16 1e-2); atol is 2e-3 (fp16 1e-3)
# where the outputs are small -- a long cache, outputs with standard deviation ~0.03 --
# and grows with the output's largest element where they are not (a few keys: outputs of
# O(1), whose rounding to 16 bits before 3d alone moves near-zero elements by ~2^-9 of
# the output's scale).
TOL_F32 = dict(rtol=1e-4, atol=1e-4)


def tol(dt, ref):
    """assert_close tolerances for a kernel storing dt, against the oracle output ref."""
    if dt == torch.float32:
        return dict(TOL_F32)
    amax = float(ref.abs().max()) if ref.numel() else 0.0
    if dt == H16:
        return dict(rtol=1e-2, atol=max(1e-3, 2.5e-3 * amax))
    return dict(rtol=2e-2, atol=max(2e-3, 1e-2 * amax))


MISTAKES = ("no_rope", "no_causal", "uniform", "scores_div4", "stale_v")
MISTAKES_FP8 = MISTAKES + ("kv_scale_twice",)


def layer_queries(g, B, Sq, H=D.n_heads):
    """(q_absorbed, q_rope) in float32 with the layer's spread (module docstring)."""
    qa = torch.randn(B, Sq, H, D.kv_rank, generator=g) * LAYER_QA_STD
    qr = torch.randn(B, Sq, H, D.rope, generator=g) * LAYER_QR_STD
    return qa, qr


def attn_inputs(B, Sq, Sk, H=D.n_heads, seed=0, dt=BF):
    """Queries with the layer's spread, a N(0,1) cache, W_uv ~ N(0, 1/kv_rank), in dt."""
    g = torch.Generator().manual_seed(seed)
    qa, qr = layer_queries(g, B, Sq, H)
    ck = torch.randn(B, Sk, D.kv_rank, generator=g)
    pe = torch.randn(B, Sk, D.rope, generator=g)
    wuv = torch.randn(H, D.v, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)
    return tuple(t.to(dt) for t in (qa, qr, ck, pe, wuv))


def fp8_inputs(B, Sq, Sk, seed):
    """bf16 queries with the layer's spread and bf16 W_uv; a N(0,1) cache quantised to e4m3
    codes of value / kv_scale with the per-tensor scale amax / 448 (the largest code)."""
    g = torch.Generator().manual_seed(seed)
    qa, qr = layer_queries(g, B, Sq)
    ck = torch.randn(B, Sk, D.kv_rank, generator=g)
    pe = torch.randn(B, Sk, D.rope, generator=g)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)
    kv_scale = float(max(ck.abs().max(), pe.abs().max())) / 448.0
    return (qa.to(BF), qr.to(BF), (ck / kv_scale).to(F8), (pe / kv_scale).to(F8), kv_scale,
            wuv.to(BF))


def paged_fp8_inputs(B, Sq, lens, page, max_pages, seed, spare=5):
    """fp8_inputs over a shuffled pool of B*max_pages + spare pages (a sequence's pages
    scattered among the others' and unused ones), one scale amax / 448 for both pools.
    Returns (qa, qr, ck_codes, pe_codes, table, seq_lens, kv_scale, wuv)."""
    g = torch.Generator().manual_seed(seed)
    n_pages = B * max_pages + spare
    table = torch.randperm(n_pages, generator=g)[:B * max_pages].reshape(B, max_pages).int()
    qa, qr = layer_queries(g, B, Sq)
    ck = torch.randn(n_pages, page, D.kv_rank, generator=g)
    pe = torch.randn(n_pages, page, D.rope, generator=g)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g) / math.sqrt(D.kv_rank)
    kv_scale = float(max(ck.abs().max(), pe.abs().max())) / 448.0
    return (qa.to(BF), qr.to(BF), (ck / kv_scale).to(F8), (pe / kv_scale).to(F8), table,
            torch.tensor(lens, dtype=torch.int32), kv_scale, wuv.to(BF))


# ---- the cases the GPU parity tests run (shared so the power test sees the same inputs)

# tests/test_gpu_fp8kv.py: dense fp8 cache, (B, Sq, Sk, causal); seed = B * 100 + Sk
FP8_DENSE_CASES = [(2, 1, 4989, False), (1, 1, 64, False), (3, 2, 1000, False),
                   (1, 8, 700, True), (1, 1, 33, False), (5, 1, 2047, False)]
FP8_FULL_SEED = 0              # the B=128, Sk=4989 case
# paged fp8 cache, (page, lens, causal, Sq); seed = page + 7 * B
FP8_PAGED_CASES = [(64, [640, 1, 333, 65], False, 1), (128, [1000, 129, 500], False, 1),
                   (64, [200, 77, 640], True, 4), (64, [0, 300, 0, 64], False, 1)]


def fp8_full_paged_lens():
    """Ragged lengths of the B=128 paged fp8 case (seed 128): in [1, 4989], the first
    sequence full, the second a single key."""
    g = torch.Generator().manual_seed(128)
    lens = torch.randint(1, 4990, (128,), generator=g).tolist()
    lens[0], lens[1] = 4989, 1
    return lens


# tests/test_gpu_flash.py: the 16-bit kernels, (B, Sq, Sk, H, causal); seed = 3 * Sk + B
FLASH16_CASES = [(1, 1, 5, 128, False), (2, 1, 33, 128, False), (3, 2, 300, 128, True),
                 (4, 1, 4989, 128, False), (2, 16, 1000, 128, True), (2, 3, 257, 40, False),
                 (1, 512, 1024, 1, True)]
# the fused-vs-oracle shapes for bf16 and fp32, (B, Sq, Sk, causal); seed = Sk + B
FUSED_CASES = [(1, 1, 1, False), (1, 1, 5, False), (2, 1, 32, False), (2, 1, 33, False),
               (3, 2, 300, True), (1, 4, 700, True), (1, 1, 4989, False), (4, 1, 4989, False),
               (2, 16, 1000, True)]


# ---- oracle variants with planted mistakes (float64, CPU)

def _stale(c):
    """Row k replaced by row k - 32 (rows below 32 kept): what a P . V stage reads when its
    ring slot still holds the previous 32-key block."""
    if c.shape[1] <= 32:
        return c
    return torch.cat([c[:, :32], c[:, :-32]], dim=1)


def attention(qa, qr, ck, pe, wuv, scale=SCALE, causal=False, mistake=None):
    """mla_attention_official in float64 on the given values, with one planted mistake
    (module docstring) or none.  [B,Sq,H,R], [B,Sq,H,D], [B,Sk,R], [B,Sk,D], [H,V,R]."""
    qa, qr, ck, pe, wuv = (t.double() for t in (qa, qr, ck, pe, wuv))
    B, Sq, H, Rk = qa.shape
    Sk = ck.shape[1]
    if mistake == "no_rope":
        qr = torch.zeros_like(qr)
    s = (torch.bmm(qa.reshape(B, Sq * H, Rk), ck.transpose(1, 2).contiguous())
         + torch.bmm(qr.reshape(B, Sq * H, -1), pe.transpose(1, 2).contiguous())) / scale
    if mistake == "scores_div4":
        s = s / 4
    if mistake == "uniform":
        s = torch.zeros_like(s)
    if causal and mistake != "no_causal":
        vis = R.causal_mask(Sq, Sk).repeat_interleave(H, dim=0)
        s = s.masked_fill(~vis.unsqueeze(0), float("-inf"))
    p = torch.softmax(s, dim=-1)
    v = _stale(ck) if mistake == "stale_v" else ck
    ctx = torch.bmm(p, v).reshape(B, Sq, H, Rk)
    return torch.einsum("bshr,hdr->bshd", ctx, wuv)


def fp8_attention(qa, qr, ck_codes, pe_codes, kv_scale, wuv, causal=False, mistake=None):
    """attention() on the decoded fp8 cache; kv_scale_twice decodes with kv_scale**2."""
    s = kv_scale * kv_scale if mistake == "kv_scale_twice" else kv_scale
    m = None if mistake == "kv_scale_twice" else mistake
    return attention(qa, qr, R.decode_e4m3(ck_codes, s), R.decode_e4m3(pe_codes, s), wuv,
                     SCALE, causal, m)


def paged_fp8_attention(qa, qr, ck_codes, pe_codes, table, seq_lens, kv_scale, wuv,
                        causal=False, mistake=None):
    """fp8_attention per sequence over its own gathered keys (an empty sequence gives zero
    rows, as in oracle.mla_ref.mla_attention_paged)."""
    B, Sq, H, _ = qa.shape
    out = torch.zeros(B, Sq, H, D.v, dtype=torch.float64)
    for b in range(B):
        n = int(seq_lens[b])
        if n == 0:
            continue
        ck = R.gather_pages(ck_codes.view(torch.uint8), table[b], n)[None]
        pe = R.gather_pages(pe_codes.view(torch.uint8), table[b], n)[None]
        out[b] = fp8_attention(qa[b:b + 1], qr[b:b + 1], ck, pe, kv_scale, wuv, causal,
                               mistake)[0]
    return out


def violates(got, want, rtol, atol):
    """True when assert_close(got, want, rtol, atol) would fail: some element with
    |got - want| > atol + rtol * |want| (or a NaN / inf mismatch)."""
    got, want = got.double(), want.double()
    if got.shape != want.shape:
        return True
    bad = (got - want).abs() > atol + rtol * want.abs()
    bad |= torch.isnan(got) != torch.isnan(want)
    return bool(bad.any())
