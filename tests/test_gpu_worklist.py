"""GPU test of the device-built ragged work list (flash_worklist_kernel) and of sequences
without keys.

* The list the kernel writes (mla_attention_work_list) for adversarial length distributions
  satisfies every invariant of tests/wl_check.py and equals the serial builder of
  worklist.h: the same chunk, slots and chunk counts, the same full items in the same
  order, and the same short items per length bucket (their order inside a bucket is the
  kernel's LDS atomics').
* seq_lens[b] = 0 gives zero output rows on both attention paths, as the oracle's softmax
  over no keys does; the other sequences of the batch are unaffected.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import wl_check as W
import attn_cases as C
from oracle import mla_ref as R

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = R.DSV3
SCALE = math.sqrt(D.qk_head)


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda
    return mla_custom_cuda


def _cases():
    rng = np.random.default_rng(5)
    Sk = 4992
    for B in (1, 7, 128, 300, 2048):
        yield B, "uniform", rng.integers(1, Sk + 1, B), Sk
        one_long = np.ones(B, dtype=np.int64)
        one_long[B // 2] = Sk
        yield B, "one_long", one_long, Sk
        yield B, "with_zeros", rng.integers(0, 3, B) * rng.integers(0, Sk + 1, B), Sk
        yield B, "all_zero", np.zeros(B, dtype=np.int64), Sk
        yield B, "equal", np.full(B, 3000), Sk
        yield B, "past_span", rng.integers(Sk - 5, 2 * Sk, B), Sk
    yield 64, "long_span", rng.integers(1, 32769, 64), 32768


CASES = list(_cases())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("Sq", [1, 4])
@pytest.mark.parametrize("case", range(len(CASES)), ids=[f"B{c[0]}-{c[1]}" for c in CASES])
def test_device_work_list(ext, dtype, Sq, case):
    B, name, lens, Sk = CASES[case]
    bk = 16 if dtype == torch.float32 else 32
    rt = W.row_tiles_of(Sq, D.n_heads)
    mi = W.max_items(B, rt)
    lens32 = torch.tensor(lens, dtype=torch.int32)
    got = ext.attention_work_list(lens32.to(DEV), Sq, D.n_heads, Sk, dtype).cpu().numpy()
    print(f"work list B={B} {name} Sq={Sq} {dtype}: {got[0]} items, chunk {got[1]}", flush=True)
    n, chunk = W.check_list(got, lens, Sk, bk, mi)
    ref = W.build_serial(lens, Sk, rt, bk)
    assert got.shape == ref.shape
    head = W.HEAD + 2 * B
    assert np.array_equal(got[:head], ref[:head]), "head, slots or chunk counts differ"
    it_g = got[head:head + 2 * n].reshape(n, 2)
    it_r = ref[head:head + 2 * n].reshape(n, 2)
    L = np.clip(lens, 0, Sk)
    nf = int(((it_r[:, 1] + 1) * chunk <= L[it_r[:, 0]]).sum())
    assert np.array_equal(it_g[:nf], it_r[:nf]), "full items differ"
    bucket = lambda it: ((chunk - 1 - L[it[:, 0]] % chunk) * W.BUCKETS) // chunk  # noqa: E731
    bg, br = bucket(it_g[nf:]), bucket(it_r[nf:])
    assert np.array_equal(bg, br), "short items fall in different buckets"
    key = lambda it, bk_: np.lexsort((it[:, 1], it[:, 0], bk_))  # noqa: E731
    assert np.array_equal(it_g[nf:][key(it_g[nf:], bg)], it_r[nf:][key(it_r[nf:], br)])


@pytest.mark.parametrize("path", ["fused", "split"])
@pytest.mark.parametrize("causal", [False, True])
def test_zero_length_sequences_give_zero_rows(ext, monkeypatch, path, causal):
    if path == "split":
        monkeypatch.setenv("MLA_ATTENTION_PATH", "split")
    else:
        monkeypatch.delenv("MLA_ATTENTION_PATH", raising=False)
    lens, page, Sq = [0, 300, 0, 65, 1000], 64, 1
    B = len(lens)
    mp = -(-max(lens) // page)
    g = torch.Generator().manual_seed(17)
    n_pages = B * mp + 2
    table = torch.randperm(n_pages, generator=g)[:B * mp].reshape(B, mp).int()
    s = 1 / math.sqrt(D.kv_rank)
    qa = torch.randn(B, Sq, D.n_heads, D.kv_rank, generator=g) * C.LAYER_QA_STD
    qr = torch.randn(B, Sq, D.n_heads, D.rope, generator=g) * C.LAYER_QR_STD
    ck = torch.randn(n_pages, page, D.kv_rank, generator=g)
    pe = torch.randn(n_pages, page, D.rope, generator=g)
    wuv = torch.randn(D.n_heads, D.v, D.kv_rank, generator=g) * s
    sl = torch.tensor(lens, dtype=torch.int32)
    out = ext.mla_attention_paged(*(t.to(DEV) for t in (qa, qr, ck, pe, table, sl, wuv)), SCALE,
                                  causal).cpu()
    assert torch.isfinite(out).all()
    ref = R.mla_attention_paged(qa, qr, ck, pe, table, sl, wuv, SCALE, causal)
    for b in (0, 2):
        assert torch.equal(out[b], torch.zeros_like(out[b])), f"sequence {b} has no keys"
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-4)
