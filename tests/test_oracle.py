"""Pin the CPU oracle (oracle/mla_ref.py) before any GPU result is compared with it.

The reference commits no golden vectors or known-answer tests, and its CUDA build and
Python oracle cannot run here.  Each oracle function is therefore pinned by checks the
mathematics fixes:

* the whole layer against an independent scalar-loop brute force (tests/brute_mla.py)
  on tiny shapes, both non-causal and causal, and against the committed fixtures that
  brute force wrote (tests/golden/*.npz);
* RoPE against the closed-form rotation, the identity at position 0 and norm
  preservation; RMSNorm against the unit-RMS property;
* the nine-step decomposition (split softmax of 3a/3b, unnormalised ctx of 3c, deferred
  divide of 3d) against the direct formulation in fp64;
* softmax normalisation, causal Sq=1 == non-causal, causal Sq=Sk == lower triangle.

``test_planted_mistakes_are_caught`` plants plausible mistakes in the oracle (a dropped
gain, swapped W_uk/W_uv, non-interleaved RoPE pairs, a multiplied scale, an off-by-one
causal limit, a dropped alpha) and shows the brute-force comparison rejects every one.
"""

from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest
import torch

import brute_mla
from oracle import mla_ref as R

TINY = R.MLADims(hidden=6, n_heads=2, q_lora=4, kv_rank=4, nope=2, rope=4, v=3)
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _brute(inp, dims, causal):
    return torch.tensor(brute_mla.layer(
        inp["x"].tolist(), inp["W_q_a"].tolist(), inp["q_norm_w"].tolist(),
        inp["W_q_b"].tolist(), inp["wkv_b"].tolist(), inp["c_kv"].tolist(),
        inp["pe_cache"].tolist(), inp["positions"].tolist(), dims.n_heads, dims.nope,
        dims.rope, dims.v, causal=causal), dtype=torch.float64)


def _oracle(inp, dims, causal):
    return R.mla_layer(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], inp["wkv_b"],
                       inp["c_kv"], inp["pe_cache"], inp["positions"], dims, causal=causal)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 3, 5), (1, 1, 7), (3, 2, 2)])
def test_layer_matches_brute_force(shape, causal):
    B, Sq, Sk = shape
    inp = R.make_inputs(B, Sq, Sk, TINY, seed=3, dtype=torch.float64)
    got = _oracle(inp, TINY, causal)
    ref = _brute(inp, TINY, causal)
    assert got.shape == (B, Sq, TINY.n_heads, TINY.v)
    torch.testing.assert_close(got, ref, rtol=1e-11, atol=1e-12)


def test_layer_matches_brute_force_large_positions():
    inp = R.make_inputs(1, 2, 6, TINY, seed=4, dtype=torch.float64)
    inp["positions"] = torch.tensor([4988, 65535], dtype=torch.int64)
    torch.testing.assert_close(_oracle(inp, TINY, False), _brute(inp, TINY, False),
                               rtol=1e-10, atol=1e-11)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))))
def test_oracle_matches_golden_fixtures(path):
    z = np.load(path)  # allow_pickle defaults to False
    B, Sq, Sk, hidden, H, q_lora, Rk, nope, rope, v, causal = [int(t) for t in z["dims"]]
    dims = R.MLADims(hidden=hidden, n_heads=H, q_lora=q_lora, kv_rank=Rk, nope=nope,
                     rope=rope, v=v)
    t = {k: torch.from_numpy(z[k]) for k in z.files if k not in ("dims", "out")}
    got = _oracle(t, dims, bool(causal))
    torch.testing.assert_close(got, torch.from_numpy(z["out"]), rtol=1e-10, atol=1e-11)
    steps = R.layer_by_steps(t, dims, causal=bool(causal), tile=4)
    torch.testing.assert_close(steps["out"], torch.from_numpy(z["out"]), rtol=1e-10,
                               atol=1e-11)


# --------------------------------------------------------------------------- RoPE


def test_rope_closed_form_rotation():
    rope = 64
    pos = torch.tensor([0, 1, 17, 4988], dtype=torch.int64)
    for i in (0, 5, 31):
        x = torch.zeros(1, len(pos), 1, rope, dtype=torch.float64)
        x[..., 2 * i] = 1.0  # unit vector on the even element of pair i
        y = R.apply_rope(x, pos, rope)
        for s, p in enumerate(pos.tolist()):
            th = p / (10000.0 ** (2 * i / rope))
            assert abs(y[0, s, 0, 2 * i].item() - math.cos(th)) < 1e-9
            assert abs(y[0, s, 0, 2 * i + 1].item() - math.sin(th)) < 1e-9
            others = torch.cat([y[0, s, 0, :2 * i], y[0, s, 0, 2 * i + 2:]])
            assert others.abs().max().item() == 0.0


def test_rope_identity_at_zero_and_norm_preserving():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 4, 64, generator=g, dtype=torch.float64)
    y0 = R.apply_rope(x, torch.zeros(3, dtype=torch.int64), 64)
    torch.testing.assert_close(y0, x, rtol=0, atol=0)
    y = R.apply_rope(x, torch.tensor([5, 900, 4988]), 64)
    n_in = x.reshape(-1, 32, 2).norm(dim=-1)
    n_out = y.reshape(-1, 32, 2).norm(dim=-1)
    torch.testing.assert_close(n_out, n_in, rtol=1e-12, atol=1e-12)


def test_rope_inv_freq_is_torch_fp32_formula():
    f = R.rope_inv_freq(64, torch.float32)
    assert f.dtype == torch.float32 and f.shape == (32,)
    assert f[0].item() == 1.0
    exact = torch.tensor([10000.0 ** (-2 * i / 64) for i in range(32)], dtype=torch.float64)
    assert (f.double() - exact).abs().max().item() < 2e-7 * 1.0


def test_step_rope_matches_apply_rope_fp64():
    B, Sq, H, nope, rope = 2, 3, 4, 8, 16
    g = torch.Generator().manual_seed(1)
    q_raw = torch.randn(B * Sq, H * (nope + rope), generator=g, dtype=torch.float64)
    pos = torch.tensor([3, 70, 4988])
    a = R.step_rope(q_raw, pos, R.rope_inv_freq(rope, torch.float64), B, Sq, H, nope, rope,
                    torch.float64)
    b = R.apply_rope(q_raw.reshape(B, Sq, H, -1)[..., nope:], pos, rope)
    torch.testing.assert_close(a, b, rtol=1e-14, atol=1e-14)


# --------------------------------------------------------------------------- RMSNorm


def test_rmsnorm_unit_rms_and_gain():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 1536, generator=g, dtype=torch.float64) * 3.0
    y = R.rmsnorm(x, torch.ones(1536, dtype=torch.float64), eps=0.0)
    torch.testing.assert_close(y.square().mean(-1), torch.ones(5, dtype=torch.float64))
    w = 1.0 + 0.1 * torch.randn(1536, generator=g, dtype=torch.float64)
    yw = R.rmsnorm(x, w, eps=0.0)
    torch.testing.assert_close(yw / w, y)
    yk = R.step_norm(x, w, 0.0, torch.float64)
    torch.testing.assert_close(yk, yw, rtol=1e-14, atol=1e-14)


# --------------------------------------------------------------------------- decomposition


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("tile", [2, 3, 128])
def test_steps_equal_direct_formulation(causal, tile):
    dims = R.MLADims(hidden=16, n_heads=4, q_lora=8, kv_rank=8, nope=4, rope=4, v=4)
    inp = R.make_inputs(2, 3, 11, dims, seed=5, dtype=torch.float64)
    steps = R.layer_by_steps(inp, dims, causal=causal, tile=tile)
    direct = _oracle(inp, dims, causal)
    torch.testing.assert_close(steps["out"], direct, rtol=1e-12, atol=1e-12)
    # the split softmax reassembles to a normalised distribution per row
    a = steps["alpha"].repeat_interleave(tile, dim=1)[:, :11]
    probs = steps["p"] * a / steps["row_sum"].unsqueeze(1)
    torch.testing.assert_close(probs.sum(-1), torch.ones(probs.shape[0], dtype=torch.float64))
    assert (steps["p"] >= 0).all() and (steps["p"] <= 1).all()


def test_causal_single_query_equals_noncausal():
    dims = R.MLADims(hidden=16, n_heads=4, q_lora=8, kv_rank=8, nope=4, rope=4, v=4)
    inp = R.make_inputs(2, 1, 9, dims, seed=6, dtype=torch.float64)
    torch.testing.assert_close(_oracle(inp, dims, True), _oracle(inp, dims, False),
                               rtol=0, atol=0)


def test_causal_mask_shape():
    m = R.causal_mask(4, 4)
    assert torch.equal(m, torch.ones(4, 4, dtype=torch.bool).tril())
    m2 = R.causal_mask(2, 5)
    assert m2.tolist() == [[True] * 4 + [False], [True] * 5]


def test_uniform_keys_give_that_key():
    dims = R.MLADims(hidden=16, n_heads=2, q_lora=8, kv_rank=8, nope=4, rope=4, v=4)
    inp = R.make_inputs(1, 1, 6, dims, seed=7, dtype=torch.float64)
    inp["c_kv"][:] = inp["c_kv"][:, :1, :]
    inp["pe_cache"][:] = inp["pe_cache"][:, :1, :]
    W_uk, W_uv = R.split_wkv_b(inp["wkv_b"], dims.nope)
    out = _oracle(inp, dims, False)
    exp = torch.einsum("r,hdr->hd", inp["c_kv"][0, 0], W_uv)
    torch.testing.assert_close(out[0, 0], exp, rtol=1e-12, atol=1e-12)


def test_make_inputs_deterministic():
    a = R.make_inputs(2, 1, 5, TINY, seed=0)
    b = R.make_inputs(2, 1, 5, TINY, seed=0)
    for k in a:
        assert torch.equal(a[k], b[k])
    assert a["positions"].tolist() == [4]
    c = R.make_inputs(2, 1, 5, TINY, seed=0, dtype=torch.bfloat16)
    assert c["x"].dtype == torch.bfloat16
    torch.testing.assert_close(c["x"].float(), a["x"], rtol=1e-2, atol=1e-2)


# --------------------------------------------------------------------------- mutants


def _mut_no_gain(mp):
    orig = R.rmsnorm
    mp.setattr(R, "rmsnorm", lambda x, g, eps=1e-6: orig(x, torch.ones_like(g), eps))


def _mut_swap_wkv(mp):
    mp.setattr(R, "split_wkv_b", lambda w, nope: (w[:, -nope:, :], w[:, :-nope, :]))


def _mut_rope_half_split(mp):
    # rotates pairs (i, i + rope/2) instead of the interleaved pairs (2i, 2i+1)
    def rope(x, positions, rope_dim):
        half = rope_dim // 2
        acc = R.acc_dtype(x.dtype)
        ang = torch.outer(positions.to(acc), R.rope_inv_freq(rope_dim, acc))
        c = torch.cos(ang).reshape(1, -1, 1, half)
        s = torch.sin(ang).reshape(1, -1, 1, half)
        a, b = x[..., :half], x[..., half:]
        return torch.cat([a * c - b * s, a * s + b * c], -1)
    mp.setattr(R, "apply_rope", rope)


def _mut_scale_multiplied(mp):
    orig = R.mla_attention_official
    mp.setattr(R, "mla_attention_official",
               lambda qa, qr, ck, pe, w, scale, causal=False: orig(qa, qr, ck, pe, w,
                                                                  1.0 / scale, causal))


def _mut_causal_off_by_one(mp):
    # key j visible iff j < Sk - Sq + i (strict), one key short of the rule
    mp.setattr(R, "causal_mask", lambda Sq, Sk: torch.arange(Sk).unsqueeze(0)
               < (Sk - Sq + torch.arange(Sq).unsqueeze(1)))


def _mut_rope_sin_sign(mp):
    orig = R.apply_rope
    mp.setattr(R, "apply_rope", lambda x, p, d: orig(x, -p, d))


MUTANTS = {
    "no_gain": _mut_no_gain,
    "swap_wkv": _mut_swap_wkv,
    "rope_half_split": _mut_rope_half_split,
    "scale_multiplied": _mut_scale_multiplied,
    "causal_off_by_one": _mut_causal_off_by_one,
    "rope_sin_sign": _mut_rope_sin_sign,
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistakes_are_caught(name, monkeypatch):
    dims = R.MLADims(hidden=6, n_heads=2, q_lora=4, kv_rank=4, nope=2, rope=4, v=2)
    causal = name == "causal_off_by_one"
    inp = R.make_inputs(2, 3, 5, dims, seed=9, dtype=torch.float64)
    inp["positions"] = torch.tensor([3, 40, 977])
    ref = _brute(inp, dims, causal)
    torch.testing.assert_close(_oracle(inp, dims, causal), ref, rtol=1e-11, atol=1e-12)
    MUTANTS[name](monkeypatch)
    bad = _oracle(inp, dims, causal)
    assert (bad - ref).abs().max().item() > 1e-6, f"mutant {name} was not detected"


def test_planted_combine_without_alpha_is_caught():
    dims = R.MLADims(hidden=16, n_heads=2, q_lora=8, kv_rank=8, nope=4, rope=4, v=4)
    inp = R.make_inputs(1, 2, 9, dims, seed=10, dtype=torch.float64)
    r = R.layer_by_steps(inp, dims, tile=2)
    W_uv = R.split_wkv_b(inp["wkv_b"], dims.nope)[1]
    ctx_bad = R.step_ctx(r["p"], torch.ones_like(r["alpha"]), inp["c_kv"], 1, 2, 2, tile=2)
    bad = R.step_out(ctx_bad, r["row_sum"], W_uv, torch.float64)
    assert (bad - _oracle(inp, dims, False)).abs().max().item() > 1e-6


# --------------------------------------------------------------------------- neighbours


def _kv_case(seed=11):
    g = torch.Generator().manual_seed(seed)
    B, Sq, hidden, Rk, D, rows, start = 2, 3, 6, 4, 4, 7, 2
    x = torch.randn(B, Sq, hidden, generator=g, dtype=torch.float64)
    W = torch.randn(hidden, Rk + D, generator=g, dtype=torch.float64) / math.sqrt(hidden)
    gain = 1.0 + 0.1 * torch.randn(Rk, generator=g, dtype=torch.float64)
    pos = torch.tensor([3, 40, 977])
    c_kv = torch.randn(B, rows, Rk, generator=g, dtype=torch.float64)
    pe = torch.randn(B, rows, D, generator=g, dtype=torch.float64)
    return x, W, gain, pos, c_kv, pe, start


def _kv_brute_check(c2, p2, x, W, gain, pos, c_kv, pe, start):
    Rk = c_kv.shape[-1]
    rows = brute_mla.kv_append(x.tolist(), W.tolist(), gain.tolist(), pos.tolist(), Rk)
    err = 0.0
    for (b, s), (crow, prow) in rows.items():
        err = max(err, (c2[b, start + s] - torch.tensor(crow, dtype=torch.float64)).abs().max().item())
        err = max(err, (p2[b, start + s] - torch.tensor(prow, dtype=torch.float64)).abs().max().item())
    Sq = x.shape[1]
    keep = [r for r in range(c_kv.shape[1]) if not start <= r < start + Sq]
    err = max(err, (c2[:, keep] - c_kv[:, keep]).abs().max().item(),
              (p2[:, keep] - pe[:, keep]).abs().max().item())
    return err


def test_kv_append_matches_brute_force():
    x, W, gain, pos, c_kv, pe, start = _kv_case()
    c2, p2 = R.kv_append(x, W, gain, pos, c_kv, pe, start, eps=1e-6)
    assert _kv_brute_check(c2, p2, x, W, gain, pos, c_kv, pe, start) < 1e-12
    # the written latent rows have unit RMS before the gain
    lat = c2[:, start:start + 3] / gain
    torch.testing.assert_close(lat.square().mean(-1), torch.ones(2, 3, dtype=torch.float64),
                               rtol=1e-5, atol=1e-5)


def _kvmut_no_gain(mp):
    orig = R.step_norm
    mp.setattr(R, "step_norm", lambda q, g, eps, dt: orig(q, torch.ones_like(g), eps, dt))


def _kvmut_rope_sign(mp):
    orig = R.step_rope
    mp.setattr(R, "step_rope", lambda q, p, f, B, Sq, H, n, r, dt: orig(q, -p, f, B, Sq, H, n, r, dt))


def _kvmut_swapped_split(mp):
    # rope on the first columns and the norm on the rest: the split of kv read backwards
    orig = R.step_gemm
    mp.setattr(R, "step_gemm", lambda a, w: orig(a, torch.roll(w, shifts=4, dims=1)))


KV_MUTANTS = {"no_gain": _kvmut_no_gain, "rope_sign": _kvmut_rope_sign,
              "swapped_split": _kvmut_swapped_split}


@pytest.mark.parametrize("name", sorted(KV_MUTANTS))
def test_kv_append_planted_mistakes_are_caught(name, monkeypatch):
    x, W, gain, pos, c_kv, pe, start = _kv_case(12)
    KV_MUTANTS[name](monkeypatch)
    c2, p2 = R.kv_append(x, W, gain, pos, c_kv, pe, start, eps=1e-6)
    assert _kv_brute_check(c2, p2, x, W, gain, pos, c_kv, pe, start) > 1e-6


def test_o_proj_matches_brute_force_and_identity():
    g = torch.Generator().manual_seed(13)
    attn = torch.randn(2, 3, 2, 3, generator=g, dtype=torch.float64)
    W = torch.randn(6, 5, generator=g, dtype=torch.float64)
    ref = torch.tensor(brute_mla.o_proj(attn.tolist(), W.tolist()), dtype=torch.float64)
    torch.testing.assert_close(R.o_proj(attn, W), ref, rtol=1e-12, atol=1e-12)
    # closed form: an identity W_o returns the heads flattened in (h, d) order
    eye = torch.eye(6, dtype=torch.float64)
    torch.testing.assert_close(R.o_proj(attn, eye), attn.reshape(2, 3, 6), rtol=0, atol=0)
    # a transposed head/dim flattening is caught
    bad = attn.permute(0, 1, 3, 2).reshape(2, 3, 6) @ W
    assert (bad - ref).abs().max().item() > 1e-6


# --------------------------------------------------------------------------- paged cache


def _paged_case(seed, B=3, Sq=2, page=4, max_pages=3, dims=None):
    dims = dims or R.MLADims(hidden=6, n_heads=2, q_lora=4, kv_rank=4, nope=2, rope=4, v=3)
    g = torch.Generator().manual_seed(seed)
    n_pages = B * max_pages + 2
    perm = torch.randperm(n_pages, generator=g)[:B * max_pages].reshape(B, max_pages).int()
    ck = torch.randn(n_pages, page, dims.kv_rank, generator=g, dtype=torch.float64)
    pe = torch.randn(n_pages, page, dims.rope, generator=g, dtype=torch.float64)
    qa = torch.randn(B, Sq, dims.n_heads, dims.kv_rank, generator=g, dtype=torch.float64)
    qr = torch.randn(B, Sq, dims.n_heads, dims.rope, generator=g, dtype=torch.float64)
    wuv = torch.randn(dims.n_heads, dims.v, dims.kv_rank, generator=g, dtype=torch.float64)
    lens = torch.tensor([max_pages * page, 5, Sq], dtype=torch.int32)[:B]
    return qa, qr, ck, pe, perm, lens, wuv


def test_gather_pages_matches_loop():
    _, _, ck, _, perm, _, _ = _paged_case(21)
    got = R.gather_pages(ck, perm[1], 10)
    for k in range(10):
        assert torch.equal(got[k], ck[int(perm[1][k // 4]), k % 4])


@pytest.mark.parametrize("causal", [False, True])
def test_paged_attention_reduces_to_dense(causal):
    """Identity table and full lengths: exactly the dense formulation on the whole batch."""
    qa, qr, _, _, _, _, wuv = _paged_case(22)
    B, page, max_pages = 3, 4, 3
    g = torch.Generator().manual_seed(23)
    dense_c = torch.randn(B, page * max_pages, 4, generator=g, dtype=torch.float64)
    dense_p = torch.randn(B, page * max_pages, 4, generator=g, dtype=torch.float64)
    table = torch.arange(B * max_pages, dtype=torch.int32).reshape(B, max_pages)
    got = R.mla_attention_paged(qa, qr, dense_c.reshape(-1, page, 4), dense_p.reshape(-1, page, 4),
                                table, torch.full((B,), page * max_pages, dtype=torch.int32),
                                wuv, 2.5, causal)
    ref = R.mla_attention_official(qa, qr, dense_c, dense_p, wuv, 2.5, causal)
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


def test_paged_attention_uses_each_length():
    """A sequence's result depends on its own keys only; one key more or less is caught."""
    qa, qr, ck, pe, perm, lens, wuv = _paged_case(24)
    got = R.mla_attention_paged(qa, qr, ck, pe, perm, lens, wuv, 2.5)
    for b in range(3):
        n = int(lens[b])
        ref = R.mla_attention_official(qa[b:b + 1], qr[b:b + 1],
                                       R.gather_pages(ck, perm[b], n)[None],
                                       R.gather_pages(pe, perm[b], n)[None], wuv, 2.5)
        torch.testing.assert_close(got[b:b + 1], ref, rtol=1e-12, atol=1e-12)
    wrong = R.mla_attention_paged(qa, qr, ck, pe, perm, lens - 1, wuv, 2.5)
    assert (wrong - got).abs().max().item() > 1e-6


def test_kv_append_paged_reduces_to_dense():
    x, W, gain, pos1, c_kv, pe, start = _kv_case(25)
    B, rows = x.shape[0], c_kv.shape[1]
    page = 7
    table = torch.arange(B, dtype=torch.int32).reshape(B, 1)   # one page of 7 rows per sequence
    pos = torch.stack([torch.arange(start, start + 3)] * B)
    c2, p2 = R.kv_append_paged(x, W, gain, pos, table, c_kv, pe, eps=1e-6)
    rc, rp = R.kv_append(x, W, gain, pos[0], c_kv, pe, start, eps=1e-6)
    torch.testing.assert_close(c2, rc, rtol=0, atol=0)
    torch.testing.assert_close(p2, rp, rtol=0, atol=0)
    assert _kv_brute_check(c2, p2, x, W, gain, pos[0], c_kv, pe, start) < 1e-12


# --------------------------------------------------------------------------- ragged Q path


def _ragged_q(inp, pos, dims=TINY):
    W_uk = R.split_wkv_b(inp["wkv_b"], dims.nope)[0]
    return R.prepare_q_ragged(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"], W_uk, pos,
                              dims.nope, dims.rope)


def test_prepare_q_ragged_matches_brute_force():
    """Per-sequence positions (distinct per row, large ones included) against the scalar
    brute force of the Q path."""
    inp = R.make_inputs(3, 2, 4, TINY, seed=31, dtype=torch.float64)
    pos = torch.tensor([[10, 11], [4987, 4988], [0, 65535]])
    qa, qr = _ragged_q(inp, pos)
    bqa, bqr = brute_mla.q_rows(inp["x"].tolist(), inp["W_q_a"].tolist(),
                                inp["q_norm_w"].tolist(), inp["W_q_b"].tolist(),
                                inp["wkv_b"].tolist(), pos.tolist(), TINY.n_heads, TINY.nope,
                                TINY.rope)
    assert qa.shape == (3, 2, TINY.n_heads, TINY.kv_rank) and qr.shape == (3, 2, TINY.n_heads,
                                                                            TINY.rope)
    torch.testing.assert_close(qa, torch.tensor(bqa, dtype=torch.float64), rtol=1e-11, atol=1e-12)
    torch.testing.assert_close(qr, torch.tensor(bqr, dtype=torch.float64), rtol=1e-10, atol=1e-11)


def test_prepare_q_ragged_equal_rows_equal_shared_positions():
    """Every sequence at the same positions: exactly the shared-positions Q path."""
    inp = R.make_inputs(4, 3, 5, TINY, seed=32, dtype=torch.float64)
    pos = inp["positions"]
    qa, qr = _ragged_q(inp, pos.unsqueeze(0).expand(4, -1))
    W_uk = R.split_wkv_b(inp["wkv_b"], TINY.nope)[0]
    sqa, sqr = R.prepare_q_mla_absorbed(inp["x"], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                                        W_uk, pos, TINY.nope, TINY.rope)
    torch.testing.assert_close(qa, sqa, rtol=0, atol=1e-14)
    torch.testing.assert_close(qr, sqr, rtol=0, atol=1e-14)


def test_prepare_q_ragged_planted_shared_row_is_caught():
    """A ragged Q path that used sequence 0's positions for every sequence is rejected."""
    inp = R.make_inputs(3, 2, 4, TINY, seed=33, dtype=torch.float64)
    pos = torch.tensor([[1, 2], [300, 301], [7, 4000]])
    good_qa, good_qr = _ragged_q(inp, pos)
    bqa, bqr = brute_mla.q_rows(inp["x"].tolist(), inp["W_q_a"].tolist(),
                                inp["q_norm_w"].tolist(), inp["W_q_b"].tolist(),
                                inp["wkv_b"].tolist(), pos.tolist(), TINY.n_heads, TINY.nope,
                                TINY.rope)
    bqr = torch.tensor(bqr, dtype=torch.float64)
    torch.testing.assert_close(good_qr, bqr, rtol=1e-10, atol=1e-11)
    bad_qa, bad_qr = _ragged_q(inp, pos[:1].expand(3, -1))
    assert (bad_qr - bqr).abs().max().item() > 1e-3


# ---- fp8 (OCP E4M3) cache ---------------------------------------------------


def test_e4m3_table_matches_torch_float8_e4m3fn():
    """The restated E4M3 decode table equals torch's own float8_e4m3fn for every code (NaN
    exactly at 0x7F and 0xFF), and spot values fixed by the format: 448 the largest,
    2^-9 the smallest subnormal, 2^-6 the smallest normal."""
    table = R.e4m3_values()
    torch_vals = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    nan = torch.isnan(table)
    assert torch.equal(nan, torch.isnan(torch_vals))
    assert nan.nonzero().flatten().tolist() == [0x7F, 0xFF]
    assert torch.equal(table[~nan], torch_vals[~nan])
    assert table[0x7E] == 448.0 and table[0x01] == 2.0 ** -9 and table[0x08] == 2.0 ** -6
    assert table[0x80] == 0.0 and math.copysign(1.0, table[0x80].item()) == -1.0


def test_e4m3_rounding_is_nearest_even():
    """torch's float8_e4m3fn conversion (how the tests build caches) rounds to the nearest
    E4M3 value, ties to the even code, checked by brute force against the table."""
    table = R.e4m3_values().double()
    finite = ~torch.isnan(table)
    grid, codes = table[finite], torch.arange(256)[finite]
    g = torch.Generator().manual_seed(3)
    x = torch.cat([torch.randn(4000, generator=g, dtype=torch.float64) * s for s in (0.01, 1, 50)])
    # exact midpoints between neighbours, which must go to the even code
    pos = torch.sort(grid[grid > 0]).values
    x = torch.cat([x, (pos[:-1] + pos[1:]) / 2])
    got = x.float().to(torch.float8_e4m3fn).view(torch.uint8).long()
    dist = (x[:, None] - grid[None, :]).abs()
    best = dist.min(dim=1).values
    for i in range(len(x)):
        cand = codes[dist[i] == best[i]].tolist()
        want = cand[0] if len(cand) == 1 else [c for c in cand if c % 2 == 0][0]
        assert got[i].item() == want or table[got[i]] == table[want], (x[i].item(), cand)


def test_fp8kv_attention_is_attention_on_the_decoded_cache():
    """mla_attention_fp8kv is mla_attention_official on code * kv_scale: a planted mistake
    (decoding without the scale) is caught."""
    g = torch.Generator().manual_seed(9)
    B, Sq, Sk, H, Rk, Dr, V = 2, 1, 40, 4, 16, 8, 8
    qa, qr = torch.randn(B, Sq, H, Rk, generator=g), torch.randn(B, Sq, H, Dr, generator=g)
    ck = (torch.randn(B, Sk, Rk, generator=g) * 3).to(torch.float8_e4m3fn)
    pe = torch.randn(B, Sk, Dr, generator=g).to(torch.float8_e4m3fn)
    wuv = torch.randn(H, V, Rk, generator=g)
    s = 0.25
    got = R.mla_attention_fp8kv(qa, qr, ck, pe, s, wuv, 3.0)
    ref = R.mla_attention_official(qa, qr, ck.float() * s, pe.float() * s, wuv, 3.0)
    torch.testing.assert_close(got, ref, rtol=1e-6, atol=1e-6)
    wrong = R.mla_attention_official(qa, qr, ck.float(), pe.float(), wuv, 3.0)
    assert (got - wrong).abs().max() > 1e-2
