"""CPU test of the ragged work list's rules (mla-cuda_amd/csrc/worklist.h).

The device builder (flash_worklist_kernel) makes every per-batch decision through the
functions of worklist.h; wl_build_serial applies them in one thread.  This test drives that
builder, built with g++, over adversarial length distributions and asserts the invariants
the fused paged pass relies on (tests/wl_check.py): at most max_items items, every
(sequence, chunk) exactly once, partial slots inside the sized range, every key covered
once.  An earlier rule without the fit check produced more items than slots for one sweep
setting and faulted the GPU; the cases with a shrunken max_items below drive that check.
"""

from __future__ import annotations

import numpy as np
import pytest

import wl_check as W

SK_FULL = 4992          # 78 pages of 64 keys, the full-size paged tests' span


def distributions(B: int, Sk: int, rng: np.random.Generator):
    yield "all_full", np.full(B, Sk)
    yield "all_one", np.ones(B, dtype=np.int64)
    yield "all_zero", np.zeros(B, dtype=np.int64)
    yield "all_mid", np.full(B, max(1, Sk // 3))
    one_long = np.ones(B, dtype=np.int64)
    one_long[B // 2] = Sk
    yield "one_long", one_long
    one_short = np.full(B, Sk)
    one_short[0] = 1
    yield "one_short", one_short
    yield "uniform", rng.integers(1, Sk + 1, B)
    yield "with_zeros", rng.integers(0, 3, B) * rng.integers(0, Sk + 1, B)
    yield "past_span", rng.integers(Sk - 5, 2 * Sk + 3, B)          # clamped to Sk
    yield "negative", rng.integers(-5, 5, B)                         # clamped to 0
    yield "alternating", np.where(np.arange(B) % 2 == 0, 0, Sk)
    yield "block_edges", rng.choice([15, 16, 17, 31, 32, 33, 63, 64, 65], B)


@pytest.mark.parametrize("B", [1, 2, 7, 64, 128, 255, 256, 257, 300, 511, 1024, 2048, 2500])
@pytest.mark.parametrize("row_tiles", [1, 2, 3, 8])
def test_work_list_invariants(B, row_tiles):
    rng = np.random.default_rng(B * 10 + row_tiles)
    for block_keys in (16, 32):
        mi = W.max_items(B, row_tiles)
        for Sk in (64, SK_FULL, 32768):
            for name, lens in distributions(B, Sk, rng):
                wl = W.build_serial(lens, Sk, row_tiles, block_keys)
                try:
                    W.check_list(wl, lens, Sk, block_keys, mi)
                except AssertionError as e:
                    raise AssertionError(f"B={B} rt={row_tiles} bk={block_keys} Sk={Sk} "
                                         f"{name}: {e}") from e


@pytest.mark.parametrize("B,shrink", [(128, 4), (300, 2), (1, 1), (2048, 3)])
def test_fit_check_doubles_the_chunk(B, shrink):
    """With fewer item slots than the chunk rule's first choice needs, the fit check
    doubles the chunk until the list fits (the rule that keeps every item and partial slot
    inside the workspace)."""
    rng = np.random.default_rng(B)
    lens = rng.integers(1, SK_FULL + 1, B)
    doubled = 0
    for row_tiles in (1, 2):
        mi = max(B + 8, W.max_items(B, row_tiles) // shrink) // 8 * 8 + 8
        wl = W.build_serial(lens, SK_FULL, row_tiles, 16, mi)
        n, chunk = W.check_list(wl, lens, SK_FULL, 16, mi)
        assert n <= mi
        n_sized, chunk_sized = W.check_list(W.build_serial(lens, SK_FULL, row_tiles, 16), lens,
                                            SK_FULL, 16, W.max_items(B, row_tiles))
        if n_sized > mi:
            assert chunk > chunk_sized, "a list over the slot count must double its chunk"
            doubled += 1
    if shrink > 1 and B < 2048:
        assert doubled, "these cases are chosen to need a doubling"


def test_equal_lengths_take_the_dense_plan():
    """Equal lengths L give the dense plan's keys per split for L, so a paged batch of equal
    lengths reproduces the dense launch (same key ranges and merge order)."""
    lib = W.harness()
    for B, rt, L, bk in [(1, 2, 4989, 16), (3, 2, 3000, 16), (128, 2, 4989, 32), (8, 2, 512, 16),
                         (300, 2, 200, 16)]:
        wl = W.build_serial(np.full(B, L), SK_FULL if L <= SK_FULL else L, rt, bk)
        assert wl[1] == lib.wl_harness_dense_keys(L, B * rt, bk)


def test_thread_partition_covers_every_batch():
    """The device builder's threads own contiguous, disjoint batch runs covering [0, B)."""
    lib = W.harness()
    for B in (1, 5, 255, 256, 257, 2048, 2049, 5000):
        firsts = [lib.wl_harness_thread_first(t, B) for t in range(257)]
        assert firsts[0] == 0 and firsts[256] == B
        assert all(a <= b for a, b in zip(firsts, firsts[1:]))


def test_checker_rejects_broken_lists():
    """The invariant checker is not vacuous: a dropped item, a doubled item and a list past
    the slot count each fail it."""
    lens = np.array([4989, 1, 2, 3, 100, 64, 65, 700])
    mi = W.max_items(8, 2)
    wl = W.build_serial(lens, SK_FULL, 2, 16)
    W.check_list(wl, lens, SK_FULL, 16, mi)
    dropped = wl.copy()
    dropped[0] -= 1
    with pytest.raises(AssertionError):
        W.check_list(dropped, lens, SK_FULL, 16, mi)
    doubled = wl.copy()
    items = doubled[W.HEAD + 16:]
    items[2:4] = items[0:2]
    with pytest.raises(AssertionError):
        W.check_list(doubled, lens, SK_FULL, 16, mi)
    with pytest.raises(AssertionError):
        W.check_list(wl, lens, SK_FULL, 16, int(wl[0]) // 8 * 8 - 8 if wl[0] > 8 else 0)


def test_dense_splits_fit_one_round_of_cus():
    """Below one workgroup per CU the dense plan takes as many key splits as fit one round:
    base x splits never passes the 256 CUs (a split count rounded to nearest once gave
    B=5, Sk=4989 260 workgroups of one per CU, and the second round's four nearly doubled
    the pass)."""
    lib = W.harness()
    for bk in (16, 32):
        for base in range(1, 256):
            for Sk in (1, 16, 64, 300, 512, 1000, 4989, 8192, 32768):
                kps = lib.wl_harness_dense_keys(Sk, base, bk)
                blocks = -(-Sk // bk)
                n_split = -(-blocks // (kps // bk))
                assert kps % bk == 0 and kps >= bk
                assert base * n_split <= 256, (bk, base, Sk, n_split)
                assert n_split <= max(1, 256 // base), (bk, base, Sk, n_split)
