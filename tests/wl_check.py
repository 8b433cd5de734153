"""Checks of the ragged work list (mla-cuda_amd/csrc/worklist.h), shared by the CPU test of
its rules and the GPU test of the device-built list.

``harness()`` builds tests/wl_harness.cpp with g++ (the header includes no HIP header) and
returns the ctypes library; ``check_list()`` asserts every invariant the fused paged pass
relies on, from the list alone and the sequence lengths:

* at most ``max_items`` items (the grid and the partial slots are sized for that many) and
  ``max_items`` a whole number per XCD (item t's row tiles are workgroups
  8 (row_tiles (t / 8) + rt) + t % 8, all inside the grid of max_items * row_tiles);
* the chunk a positive multiple of the key block;
* sequence b has max(1, ceil(L_b / chunk)) chunks whose key ranges cover [0, L_b) exactly
  once, with L_b = seq_lens[b] clamped to [0, Sk];
* partial slots batch-major, disjoint, inside [0, max_items);
* every (b, c) listed exactly once; full-length chunks before the shorter last chunks, and
  those in non-increasing length order (up to the bucket width).
"""

from __future__ import annotations

import ctypes
import os
import shutil
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "mla-cuda_amd", "csrc")
HEAD = 2
BUCKETS = 256

_LIB = None


def harness():
    """The g++-built harness library (built once per process into a temporary folder)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    gxx = shutil.which("g++")
    if gxx is None:
        raise RuntimeError("g++ not found: the work-list harness cannot be built")
    out = os.path.join(tempfile.mkdtemp(prefix="wl_harness_"), "libwl_harness.so")
    subprocess.run([gxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Werror",
                    "-I", CSRC, os.path.join(HERE, "wl_harness.cpp"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    ip = ctypes.POINTER(ctypes.c_int)
    lib.wl_harness_build.argtypes = [ip, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ip]
    for f in ("wl_harness_max_items", "wl_harness_ints", "wl_harness_bucket",
              "wl_harness_thread_first"):
        getattr(lib, f).argtypes = [ctypes.c_int, ctypes.c_int]
    lib.wl_harness_dense_keys.argtypes = [ctypes.c_int] * 3
    _LIB = lib
    return lib


def row_tiles_of(Sq: int, H: int) -> int:
    return -(-Sq * H // 64)


def max_items(B: int, row_tiles: int) -> int:
    return harness().wl_harness_max_items(B, row_tiles)


def build_serial(lens, Sk: int, row_tiles: int, block_keys: int, mi: int | None = None):
    """The list as wl_build_serial makes it (np.int32 array of wl_ints(B, max_items))."""
    lib = harness()
    lens = np.ascontiguousarray(np.asarray(lens, dtype=np.int32))
    B = len(lens)
    if mi is None:
        mi = lib.wl_harness_max_items(B, row_tiles)
    wl = np.full(lib.wl_harness_ints(B, mi), -7, dtype=np.int32)
    ip = ctypes.POINTER(ctypes.c_int)
    lib.wl_harness_build(lens.ctypes.data_as(ip), B, Sk, row_tiles, block_keys, mi,
                         wl.ctypes.data_as(ip))
    return wl


def check_list(wl, lens, Sk: int, block_keys: int, mi: int):
    """Assert every invariant of a work list (see the module docstring)."""
    wl = np.asarray(wl, dtype=np.int64)
    lens = np.clip(np.asarray(lens, dtype=np.int64), 0, Sk)
    B = len(lens)
    n, chunk = int(wl[0]), int(wl[1])
    assert mi % 8 == 0, f"max_items {mi} not a whole number per XCD"
    assert 0 < n <= mi, f"{n} items for {mi} slots"
    assert chunk > 0 and chunk % block_keys == 0, f"chunk {chunk}"
    first = wl[HEAD:HEAD + B]
    count = wl[HEAD + B:HEAD + 2 * B]
    items = wl[HEAD + 2 * B:HEAD + 2 * B + 2 * n].reshape(n, 2)
    want = np.maximum(1, -(-lens // chunk))
    assert np.array_equal(count, want), "chunk counts"
    assert int(count.sum()) == n, "item count"
    assert np.array_equal(first, np.concatenate([[0], np.cumsum(count)[:-1]])), "slots"
    assert int((first + count).max()) <= mi, "partial slot past the sized range"
    # every (b, c) exactly once
    keys = items[:, 0] * (int(count.max()) + 1) + items[:, 1]
    assert np.all((items[:, 0] >= 0) & (items[:, 0] < B)), "batch index"
    assert np.all((items[:, 1] >= 0) & (items[:, 1] < count[items[:, 0]])), "chunk index"
    assert len(np.unique(keys)) == n, "an item is listed twice"
    # the chunks of each sequence cover its keys exactly once
    lo = items[:, 1] * chunk
    hi = np.minimum(lo + chunk, lens[items[:, 0]])
    covered = np.zeros(B, dtype=np.int64)
    np.add.at(covered, items[:, 0], np.maximum(0, hi - lo))
    assert np.array_equal(covered, lens), "keys covered"
    # dispatch order: full chunks first, then the short ones longest first
    full = (items[:, 1] + 1) * chunk <= lens[items[:, 0]]
    nf = int(full.sum())
    assert full[:nf].all() and not full[nf:].any(), "full chunks first"
    rem = lens[items[nf:, 0]] % chunk
    bucket = ((chunk - 1 - rem) * BUCKETS) // chunk
    assert np.all(np.diff(bucket) >= 0), "short chunks longest first"
    return n, chunk
