"""CPU-only checks of the drop-in boundary: the C ABI library and the torch binding.

No test here launches device work.  Every call below is rejected by argument validation,
which the C ABI performs completely before its first HIP call (so these run on a machine
without a GPU), or is a pure host query (workspace sizes, score layout).
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mla", "mla.h")
LIB = os.path.join(ROOT, "mla-cuda_amd", "libmla_amd.so")

MLA_OK, MLA_ERR_INVALID_ARGUMENT, MLA_ERR_UNSUPPORTED, MLA_ERR_WORKSPACE, MLA_ERR_HIP = range(5)
F32, BF16 = 0, 1


class Dims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("batch", "sq", "sk", "hidden", "q_lora", "heads", "nope", "rope", "kv_rank", "v")]


def dsv3(B=1, Sq=1, Sk=512):
    return Dims(B, Sq, Sk, 7168, 1536, 128, 128, 64, 512, 128)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(LIB)
    L.mla_last_error.restype = ctypes.c_char_p
    L.mla_version.restype = ctypes.c_char_p
    for n in ("mla_q_absorbed_workspace_bytes", "mla_attention_workspace_bytes",
              "mla_gemm_workspace_bytes", "mla_ctx_workspace_bytes", "mla_out_workspace_bytes",
              "mla_attention_streaming_workspace_bytes", "mla_kv_append_workspace_bytes",
              "mla_o_proj_workspace_bytes", "mla_attention_paged_workspace_bytes",
              "mla_attn_ctx_workspace_bytes"):
        getattr(L, n).restype = ctypes.c_size_t
    return L


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mla_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = header_functions()
    for must in ("mla_q_absorbed", "mla_attention", "mla_gemm", "mla_rmsnorm", "mla_rope",
                 "mla_absorb", "mla_scores", "mla_combine", "mla_ctx", "mla_out",
                 "mla_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), f"{name} declared in mla.h but not exported"


def test_library_exports_only_the_abi():
    out = os.popen(f"nm -D --defined-only {LIB}").read()
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == set(header_functions())


def test_version_and_layout_queries(lib):
    assert b"gfx950" in lib.mla_version()
    assert lib.mla_score_tile() == 128
    assert lib.mla_score_ld(4989) == 4992
    assert lib.mla_score_ld(32) == 32 and lib.mla_score_ld(33) == 64
    assert lib.mla_score_ld(0) == 0


def test_workspace_queries_are_pure_host(lib, monkeypatch):
    d = dsv3(128, 1, 4989)
    wq = lib.mla_q_absorbed_workspace_bytes(F32, ctypes.byref(d))
    rows = 128 * 128
    # fused path (the default at these widths): ctx, row sums, 3d's workspace -- no scores
    wa = lib.mla_attention_workspace_bytes(F32, ctypes.byref(d), 0)
    assert rows * 512 * 4 <= wa < rows * 512 * 4 * 1.5
    # per-step path: scores [rows, 4992] fp32 alone is 327 MB
    monkeypatch.setenv("MLA_ATTENTION_PATH", "split")
    ws = lib.mla_attention_workspace_bytes(F32, ctypes.byref(d), 0)
    assert ws >= rows * 4992 * 4 + rows * 512 * 4
    assert ws < rows * 4992 * 4 * 1.3
    monkeypatch.delenv("MLA_ATTENTION_PATH")
    # q path: q_lat, q_raw at least
    assert wq >= 128 * (1536 + 128 * 192) * 4
    bad = dsv3(0, 1, 4989)
    assert lib.mla_attention_workspace_bytes(F32, ctypes.byref(bad), 0) == 0


def _err(lib):
    return lib.mla_last_error().decode()


P16 = ctypes.c_void_p(1 << 20)   # aligned fake device pointer (never dereferenced)
P_ODD = ctypes.c_void_p((1 << 20) + 4)


def test_gemm_validation(lib):
    st = lib.mla_gemm(F32, P16, P16, P16, 0, 16, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "M must be positive" in _err(lib)
    st = lib.mla_gemm(F32, P16, P16, P16, 4, 18, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "N must be a positive multiple of 4" in _err(lib)
    st = lib.mla_gemm(F32, None, P16, P16, 4, 16, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "A must not be NULL" in _err(lib)
    st = lib.mla_gemm(F32, P_ODD, P16, P16, 4, 16, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "16-byte aligned" in _err(lib)
    st = lib.mla_gemm(7, P16, P16, P16, 4, 16, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "unknown dtype" in _err(lib)


def test_fp16_is_a_storage_dtype(lib):
    """MLA_DTYPE_F16 (2) passes the dtype check and takes the 16-bit row rule (multiples
    of 8 elements), like bf16; the next code is still unknown."""
    st = lib.mla_gemm(2, P16, P16, P16, 0, 16, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "M must be positive" in _err(lib)
    st = lib.mla_gemm(2, P16, P16, P16, 4, 20, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "multiple of 8 for fp16" in _err(lib)
    st = lib.mla_gemm(4, P16, P16, P16, 4, 16, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "unknown dtype" in _err(lib)


F64 = 3


def test_fp64_is_taken_by_the_fused_entry_points_only(lib):
    """MLA_DTYPE_F64 (3): the two fused entry points (and the no-workspace attention) size a
    double workspace -- the [B*Sq*H, Sk] score matrix plus ctx, or the Q path's q_lat and
    q_raw -- and every other entry point refuses it (MLA_ERR_UNSUPPORTED) before touching
    the device."""
    d = dsv3(B=1, Sq=1, Sk=64)
    ws = lib.mla_attention_workspace_bytes(F64, ctypes.byref(d), 0)
    rows = 128
    assert ws >= rows * 64 * 8 + rows * 512 * 8
    assert ws < rows * 64 * 8 + rows * 512 * 8 + 4096
    wq = lib.mla_q_absorbed_workspace_bytes(F64, ctypes.byref(d))
    assert wq >= 1536 * 8 + 128 * 192 * 8
    st = lib.mla_gemm(F64, P16, P16, P16, 4, 16, 16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_UNSUPPORTED and "float64" in _err(lib)
    lib.mla_attention_fp8kv_workspace_bytes.restype = ctypes.c_size_t
    assert lib.mla_attention_fp8kv_workspace_bytes(F64, ctypes.byref(d), 0) == 0
    assert lib.mla_attention_streaming_workspace_bytes(F64, ctypes.byref(d), 0, 0) == 0
    st = lib.mla_attention_streaming(F64, ctypes.byref(d), P16, P16, P16, P16, P16,
                                     ctypes.c_double(13.85), 0, 0, P16, P16,
                                     ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_UNSUPPORTED and "float64" in _err(lib)
    st = lib.mla_rope(F64, ctypes.byref(d), P16, P16, P16, P16, None)
    assert st == MLA_ERR_UNSUPPORTED
    # the f64 shape rules: positive dims, an even rope width; rejected before any HIP call
    bad = dsv3(B=1, Sq=1, Sk=64)
    bad.rope = 7
    assert lib.mla_q_absorbed_workspace_bytes(F64, ctypes.byref(bad)) == 0
    st = lib.mla_q_absorbed(F64, ctypes.byref(bad), P16, P16, P16, P16, P16, P16, P16,
                            ctypes.c_double(1e-6), P16, P16, P16, ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "rope" in _err(lib)
    st = lib.mla_attention(F64, ctypes.byref(d), P16, P16, P16, P16, P16, ctypes.c_double(13.85),
                           0, P16, P16, ctypes.c_size_t(ws - 1), None)
    assert st == MLA_ERR_WORKSPACE
    st = lib.mla_attention(F64, ctypes.byref(d), P16, P_ODD, P16, P16, P16,
                           ctypes.c_double(13.85), 0, P16, P16, ctypes.c_size_t(ws), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "aligned" in _err(lib)
    causal = dsv3(B=1, Sq=8, Sk=4)
    assert lib.mla_attention_workspace_bytes(F64, ctypes.byref(causal), 1) == 0


def test_fp8kv_validation(lib):
    """The fp8-cache attention takes bf16 queries only and a positive finite kv_scale, and
    sizes a workspace for the DeepSeek-V3 widths."""
    dims = Dims(2, 1, 64, 7168, 1536, 128, 128, 64, 512, 128)
    lib.mla_attention_fp8kv_workspace_bytes.restype = ctypes.c_size_t
    assert lib.mla_attention_fp8kv_workspace_bytes(1, ctypes.byref(dims), 0) > 0
    assert lib.mla_attention_fp8kv_workspace_bytes(0, ctypes.byref(dims), 0) == 0
    call = lambda dt, s: lib.mla_attention_fp8kv(  # noqa: E731
        dt, ctypes.byref(dims), P16, P16, P16, P16, ctypes.c_float(s), P16, ctypes.c_double(1.0),
        0, P16, None, ctypes.c_size_t(0), None)
    assert call(0, 1.0) == MLA_ERR_UNSUPPORTED and "bf16 queries" in _err(lib)
    assert call(1, 0.0) == MLA_ERR_INVALID_ARGUMENT and "kv_scale" in _err(lib)
    assert call(1, float("inf")) == MLA_ERR_INVALID_ARGUMENT


def test_fp8kv_refuses_query_spans_past_32_bit_offsets(lib):
    """The fused fp8 pass forms 32-bit buffer offsets within a sequence's query rows (bf16,
    1 KiB each) and has no per-step path to fall back on: Sq * heads * 1 KiB >= 2^31 is
    refused (UNSUPPORTED, zero workspace), dense and paged, where bf16 at the same shape
    falls back to the split path.  One query row less than the limit is accepted."""
    lib.mla_attention_fp8kv_workspace_bytes.restype = ctypes.c_size_t
    lib.mla_attention_paged_fp8kv_workspace_bytes.restype = ctypes.c_size_t
    big = Dims(1, 16384, 64, 7168, 1536, 128, 128, 64, 512, 128)     # 2 GiB of query rows
    assert lib.mla_attention_fp8kv_workspace_bytes(1, ctypes.byref(big), 0) == 0
    assert lib.mla_attention_paged_fp8kv_workspace_bytes(1, ctypes.byref(big), 0, 64) == 0
    st = lib.mla_attention_fp8kv(1, ctypes.byref(big), P16, P16, P16, P16, ctypes.c_float(1.0),
                                 P16, ctypes.c_double(13.85), 0, P16, P16,
                                 ctypes.c_size_t(1 << 40), None)
    assert st == MLA_ERR_UNSUPPORTED and "2^31" in _err(lib)
    st = lib.mla_attention_paged_fp8kv(1, ctypes.byref(big), P16, P16, P16, P16, P16, P16, 64,
                                       ctypes.c_float(1.0), P16, ctypes.c_double(13.85), 0, P16,
                                       P16, ctypes.c_size_t(1 << 40), None)
    assert st == MLA_ERR_UNSUPPORTED and "2^31" in _err(lib)
    # the bf16 path at the same shape still plans (on the per-step kernels)
    assert lib.mla_attention_workspace_bytes(1, ctypes.byref(big), 0) > 0
    ok = Dims(1, 16383, 16384, 7168, 1536, 128, 128, 64, 512, 128)   # 2^31 - 128 KiB
    assert lib.mla_attention_fp8kv_workspace_bytes(1, ctypes.byref(ok), 0) > 0


def test_paged_fp8kv_validation(lib):
    """The paged fp8-cache attention takes the fp8 rules (bf16 queries, a positive finite
    kv_scale) and the page rules (page_size a positive multiple of 64 dividing dims.sk), and
    sizes its workspace like the dense fp8 call plus the work list and its partial slots."""
    d = Dims(128, 1, 4992, 7168, 1536, 128, 128, 64, 512, 128)
    lib.mla_attention_paged_fp8kv_workspace_bytes.restype = ctypes.c_size_t
    lib.mla_attention_fp8kv_workspace_bytes.restype = ctypes.c_size_t
    ws = lib.mla_attention_paged_fp8kv_workspace_bytes(1, ctypes.byref(d), 0, 64)
    dense = lib.mla_attention_fp8kv_workspace_bytes(1, ctypes.byref(d), 0)
    row_tiles, B = 2, 128
    items = -(-(4 * 256 // row_tiles + B + 1) // 8) * 8
    extra = items * 128 * (512 + 2) * 4 + (2 + 2 * B + 2 * items) * 4
    assert dense > 0 and dense < ws <= dense + extra + 4096
    assert lib.mla_attention_paged_fp8kv_workspace_bytes(0, ctypes.byref(d), 0, 64) == 0
    assert lib.mla_attention_paged_fp8kv_workspace_bytes(1, ctypes.byref(d), 0, 96) == 0
    call = lambda dt, page, s, lens=P16: lib.mla_attention_paged_fp8kv(  # noqa: E731
        dt, ctypes.byref(d), P16, P16, P16, P16, P16, lens, page, ctypes.c_float(s), P16,
        ctypes.c_double(13.85), 0, P16, P16, ctypes.c_size_t(ws), None)
    assert call(0, 64, 1.0) == MLA_ERR_UNSUPPORTED and "bf16 queries" in _err(lib)
    assert call(1, 64, 0.0) == MLA_ERR_INVALID_ARGUMENT and "kv_scale" in _err(lib)
    assert call(1, 100, 1.0) == MLA_ERR_INVALID_ARGUMENT and "page_size" in _err(lib)
    assert call(1, 64, 1.0, None) == MLA_ERR_INVALID_ARGUMENT and "seq_lens must not be NULL" in _err(lib)
    d.sk = 4989
    assert call(1, 64, 1.0) == MLA_ERR_INVALID_ARGUMENT and "max_pages * page_size" in _err(lib)


def test_gemm_split_needs_workspace(lib):
    need = lib.mla_gemm_workspace_bytes(F32, 1, 1536, 7168)
    assert need > 0, "B=1 2a1 is split over K"
    st = lib.mla_gemm(F32, P16, P16, P16, 1, 1536, 7168, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_WORKSPACE and "workspace is NULL" in _err(lib)
    st = lib.mla_gemm(F32, P16, P16, P16, 1, 1536, 7168, P16, ctypes.c_size_t(need - 1), None)
    assert st == MLA_ERR_WORKSPACE and "too small" in _err(lib)


def test_weight_streaming_plans_size_the_workspace(lib, monkeypatch):
    """The 16-bit B=128 projections take the weight-streaming plans: 2a1 in 8 K splits
    (fp32 partials [8][128][1536]), 2a2 unsplit (no workspace).  MLA_WGEMM=0 returns the
    tiled engine's plans, whose workspace the query reports as well; MLA_WGEMM_PLAN
    forces a plan, and a plan the engine cannot run (N % bn != 0) falls back to the
    tiled one."""
    assert lib.mla_gemm_workspace_bytes(BF16, 128, 1536, 7168) == 8 * 128 * 1536 * 4
    assert lib.mla_gemm_workspace_bytes(BF16, 128, 24576, 1536) == 0
    monkeypatch.setenv("MLA_WGEMM_PLAN", "128,24576,1536,1=128,3")
    assert lib.mla_gemm_workspace_bytes(BF16, 128, 24576, 1536) == 3 * 128 * 24576 * 4
    monkeypatch.setenv("MLA_WGEMM_PLAN", "40,200,128,1=128,1")
    tiled = lib.mla_gemm_workspace_bytes(BF16, 40, 200, 128)
    monkeypatch.setenv("MLA_WGEMM", "0")
    assert lib.mla_gemm_workspace_bytes(BF16, 40, 200, 128) == tiled


def test_attention_validation(lib):
    d = dsv3(2, 3, 2)
    args = [P16] * 5
    st = lib.mla_attention(F32, ctypes.byref(d), *args, ctypes.c_double(13.85), 1, P16, P16,
                           ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "sk >= sq" in _err(lib)
    d = dsv3(2, 1, 100)
    st = lib.mla_attention(F32, ctypes.byref(d), *args, ctypes.c_double(0.0), 0, P16, P16,
                           ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "scale" in _err(lib)
    st = lib.mla_attention(F32, ctypes.byref(d), *args, ctypes.c_double(13.85), 0, P16, None,
                           ctypes.c_size_t(0), None)
    assert st == MLA_ERR_WORKSPACE
    d.kv_rank = 510
    st = lib.mla_attention(F32, ctypes.byref(d), *args, ctypes.c_double(13.85), 0, P16, P16,
                           ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "kv_rank" in _err(lib)
    st = lib.mla_attention(F32, None, *args, ctypes.c_double(13.85), 0, P16, P16,
                           ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "dims" in _err(lib)


def test_attn_ctx_validation_and_workspace(lib):
    """The fused 3a+3b+3c entry point: kv_rank 512 / rope 64 only (bf16 or fp32); its
    workspace is the split partials (a scratch row when one split covers the keys)."""
    d = dsv3(128, 1, 4989)
    for dt in (F32, BF16):
        ws = lib.mla_attn_ctx_workspace_bytes(dt, ctypes.byref(d), 0)
        assert 0 < ws <= 128 * 128 * 4 + 256      # one split: the row-maximum scratch only
    d1 = dsv3(1, 1, 4989)
    ws1 = lib.mla_attn_ctx_workspace_bytes(BF16, ctypes.byref(d1), 0)
    assert ws1 >= 2 * 128 * (512 + 2) * 4          # several splits: partial ctx, m, l
    assert lib.mla_attn_ctx_workspace_bytes(F32, ctypes.byref(d1), 0) >= 2 * 128 * 514 * 4
    args = [P16] * 4
    d.kv_rank = 256
    assert lib.mla_attn_ctx_workspace_bytes(F32, ctypes.byref(d), 0) == 0
    st = lib.mla_attn_ctx(F32, ctypes.byref(d), *args, ctypes.c_double(13.85), 0, P16, P16,
                          P16, ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_UNSUPPORTED and "kv_rank 512" in _err(lib)
    st = lib.mla_attn_ctx(BF16, ctypes.byref(d), *args, ctypes.c_double(13.85), 0, P16, P16,
                          P16, ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_UNSUPPORTED
    d = dsv3(2, 3, 2)
    st = lib.mla_attn_ctx(BF16, ctypes.byref(d), *args, ctypes.c_double(13.85), 1, P16, P16,
                          P16, ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "sk >= sq" in _err(lib)
    d = dsv3(1, 1, 4989)
    st = lib.mla_attn_ctx(BF16, ctypes.byref(d), *args, ctypes.c_double(13.85), 0, P16, P16,
                          P16, ctypes.c_size_t(ws1 - 1), None)
    assert st == MLA_ERR_WORKSPACE and "too small" in _err(lib)


def test_q_absorbed_validation(lib):
    d = dsv3(1, 1, 1)
    d.rope = 6
    ptrs = [P16] * 7
    st = lib.mla_q_absorbed(F32, ctypes.byref(d), *ptrs, ctypes.c_double(1e-6), P16, P16, P16,
                            ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "rope" in _err(lib)
    d.rope = 64
    st = lib.mla_q_absorbed(F32, ctypes.byref(d), *ptrs, ctypes.c_double(-1.0), P16, P16, P16,
                            ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "eps" in _err(lib)


def test_bf16_needs_8_element_rows(lib):
    d = dsv3(1, 1, 100)
    d.rope = 68
    st = lib.mla_attention(BF16, ctypes.byref(d), *([P16] * 5), ctypes.c_double(13.85), 0, P16,
                           P16, ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "multiple of 8 for bf16" in _err(lib)
    assert lib.mla_attention_workspace_bytes(BF16, ctypes.byref(dsv3(2, 1, 100)), 0) > 0


def test_streaming_validation_and_bounded_workspace(lib, monkeypatch):
    d = dsv3(4, 128, 32768)
    fused = lib.mla_attention_workspace_bytes(F32, ctypes.byref(d), 1)
    monkeypatch.setenv("MLA_ATTENTION_PATH", "split")
    full = lib.mla_attention_workspace_bytes(F32, ctypes.byref(d), 1)
    monkeypatch.delenv("MLA_ATTENTION_PATH")
    stream = lib.mla_attention_streaming_workspace_bytes(F32, ctypes.byref(d), 1, 0)
    assert full > 8.5e9            # the materialised [65536 x 32768] fp32 scores
    assert 0 < stream < 1.6e9      # one <= 1 GiB chunk of scores plus the running state
    assert 0 < fused < 0.2e9       # the fused pass keeps no scores: ctx and row sums
    small = lib.mla_attention_streaming_workspace_bytes(F32, ctypes.byref(d), 1, 128)
    assert 0 < small < stream
    assert lib.mla_attention_streaming_workspace_bytes(F32, ctypes.byref(d), 1, 100) == 0
    st = lib.mla_attention_streaming(F32, ctypes.byref(d), *([P16] * 5), ctypes.c_double(13.85),
                                     1, 100, P16, P16, ctypes.c_size_t(1 << 31), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "key_chunk" in _err(lib)
    st = lib.mla_attention_streaming(F32, ctypes.byref(d), *([P16] * 5), ctypes.c_double(13.85),
                                     1, 0, P16, P16, ctypes.c_size_t(stream - 1), None)
    assert st == MLA_ERR_WORKSPACE


def test_scores_validation(lib):
    d = dsv3(1, 1, 100)
    st = lib.mla_scores(F32, ctypes.byref(d), P16, P16, P16, P16, ctypes.c_double(13.8), 0,
                        P16, 100, P16, P16, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "ld_scores" in _err(lib)


def test_split_wkv_b_validation(lib):
    d = dsv3()
    st = lib.mla_split_wkv_b(F32, ctypes.byref(d), P16, P16, None, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "W_uv must not be NULL" in _err(lib)
    d.v = 0
    st = lib.mla_split_wkv_b(F32, ctypes.byref(d), P16, P16, P16, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "dims.v" in _err(lib)
    d = dsv3()
    d.kv_rank = 500
    st = lib.mla_split_wkv_b(BF16, ctypes.byref(d), P16, P16, P16, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "multiple of 8 for bf16" in _err(lib)


def test_kv_append_validation_and_workspace(lib):
    d = dsv3(128, 1, 4989)
    need = lib.mla_kv_append_workspace_bytes(F32, ctypes.byref(d))
    assert need >= 128 * 576 * 4, "x @ W_kv_a lands in the workspace"
    ptrs = [P16] * 5
    st = lib.mla_kv_append(F32, ctypes.byref(d), *ptrs, ctypes.c_double(1e-6), 4989, 4989, P16,
                           P16, P16, ctypes.c_size_t(need), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "start_row" in _err(lib)
    st = lib.mla_kv_append(F32, ctypes.byref(d), *ptrs, ctypes.c_double(float("nan")), 0, 4989,
                           P16, P16, P16, ctypes.c_size_t(need), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "eps" in _err(lib)
    st = lib.mla_kv_append(F32, ctypes.byref(d), *ptrs, ctypes.c_double(1e-6), 4988, 4989, P16,
                           P16, P16, ctypes.c_size_t(need - 1), None)
    assert st == MLA_ERR_WORKSPACE
    st = lib.mla_kv_append(F32, ctypes.byref(d), *ptrs, ctypes.c_double(1e-6), 4988, 4989, P16,
                           None, P16, ctypes.c_size_t(need), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "pe_cache must not be NULL" in _err(lib)


def test_o_proj_validation_and_workspace(lib):
    d = dsv3(128, 1, 1)
    need = lib.mla_o_proj_workspace_bytes(F32, ctypes.byref(d))
    assert need > 0, "K = H*v = 16384 against 56 output tiles is split over K"
    st = lib.mla_o_proj(F32, ctypes.byref(d), P16, P16, P16, None, ctypes.c_size_t(0), None)
    assert st == MLA_ERR_WORKSPACE
    d.hidden = 7166
    st = lib.mla_o_proj(F32, ctypes.byref(d), P16, P16, P16, P16, ctypes.c_size_t(need), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "dims.hidden" in _err(lib)


def test_paged_validation(lib, monkeypatch):
    d = dsv3(128, 1, 4992)
    ws = lib.mla_attention_paged_workspace_bytes(F32, ctypes.byref(d), 0, 64)
    dense = lib.mla_attention_workspace_bytes(F32, ctypes.byref(d), 0)
    # the fused paged pass adds the work list and the partial slots of its balanced grid:
    # at most 4 * 256 / row_tiles + B + 1 items (rounded up to a multiple of the 8 XCDs)
    # of 128 rows x (512 + 2) floats, plus the list
    row_tiles, B = 2, 128
    items = -(-(4 * 256 // row_tiles + B + 1) // 8) * 8
    extra = items * 128 * (512 + 2) * 4 + (2 + 2 * B + 2 * items) * 4
    assert dense > 0 and dense < ws <= dense + extra + 4096
    monkeypatch.setenv("MLA_ATTENTION_PATH", "split")   # the per-step path: same layout
    assert (lib.mla_attention_paged_workspace_bytes(F32, ctypes.byref(d), 0, 64) ==
            lib.mla_attention_workspace_bytes(F32, ctypes.byref(d), 0))
    monkeypatch.delenv("MLA_ATTENTION_PATH")
    assert lib.mla_attention_paged_workspace_bytes(F32, ctypes.byref(d), 0, 96) == 0
    args = [P16] * 6
    st = lib.mla_attention_paged(F32, ctypes.byref(d), *args, 100, P16, ctypes.c_double(13.85), 0,
                                 P16, P16, ctypes.c_size_t(ws), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "page_size" in _err(lib)
    d.sk = 4989
    st = lib.mla_attention_paged(F32, ctypes.byref(d), *args, 64, P16, ctypes.c_double(13.85), 0,
                                 P16, P16, ctypes.c_size_t(ws), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "max_pages * page_size" in _err(lib)
    d.sk = 4992
    st = lib.mla_attention_paged(F32, ctypes.byref(d), P16, P16, P16, P16, P16, None, 64, P16,
                                 ctypes.c_double(13.85), 0, P16, P16, ctypes.c_size_t(ws), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "seq_lens must not be NULL" in _err(lib)
    st = lib.mla_kv_append_paged(F32, ctypes.byref(d), *([P16] * 5), ctypes.c_double(1e-6), None,
                                 64, P16, P16, P16, ctypes.c_size_t(1 << 30), None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "block_table must not be NULL" in _err(lib)


# ------------------------------------------------------------------ torch binding


@pytest.fixture(scope="module")
def ext():
    import mla_custom_cuda
    return mla_custom_cuda


def test_binding_surface(ext):
    for name in ("q_absorbed", "mla_attention", "gemm", "rmsnorm", "rope", "absorb", "scores",
                 "combine", "ctx", "out", "rope_inv_freq", "attn_ctx"):
        assert callable(getattr(ext, name))


def test_binding_inv_freq_matches_oracle_bitwise(ext):
    from oracle import mla_ref as R
    for rope in (64, 16, 128):
        assert torch.equal(ext.rope_inv_freq(rope), R.rope_inv_freq(rope, torch.float32))
        f64 = ext.rope_inv_freq(rope, float64=True)
        assert f64.dtype == torch.float64
        assert torch.equal(f64, R.rope_inv_freq(rope, torch.float64))


def _attn(B=1, Sq=1, Sk=8, H=4, Rk=16, D=8, V=8, dtype=torch.float32):
    return (torch.zeros(B, Sq, H, Rk, dtype=dtype), torch.zeros(B, Sq, H, D, dtype=dtype),
            torch.zeros(B, Sk, Rk, dtype=dtype), torch.zeros(B, Sk, D, dtype=dtype),
            torch.zeros(H, V, Rk, dtype=dtype))


def test_binding_attention_shape_errors(ext):
    qa, qr, ck, pe, wuv = _attn()
    with pytest.raises(RuntimeError, match="c_kv must be"):
        ext.mla_attention(qa, qr, ck[:, :, :8], pe, wuv, 1.0)
    with pytest.raises(RuntimeError, match="pe_cache must be"):
        ext.mla_attention(qa, qr, ck, pe[:, :4], wuv, 1.0)
    with pytest.raises(RuntimeError, match="W_uv must be"):
        ext.mla_attention(qa, qr, ck, pe, wuv[:2], 1.0)
    with pytest.raises(RuntimeError, match="q_absorbed must be"):
        ext.mla_attention(qa[0], qr, ck, pe, wuv, 1.0)
    with pytest.raises(RuntimeError, match="dtype"):
        ext.mla_attention(qa.int(), qr.int(), ck.int(), pe.int(), wuv.int(), 1.0)
    with pytest.raises(RuntimeError, match="c_kv has dtype"):
        ext.mla_attention(qa.double(), qr.double(), ck, pe.double(), wuv.double(), 1.0)
    with pytest.raises(RuntimeError, match="c_kv has dtype"):
        ext.mla_attention(qa, qr, ck.bfloat16(), pe, wuv, 1.0)
    with pytest.raises(RuntimeError, match="causal attention needs Sk >= Sq"):
        a = _attn(Sq=9, Sk=8)
        ext.mla_attention(*a, 1.0, True)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        ext.mla_attention(qa, qr, ck, pe, wuv, 1.0)


def test_binding_q_absorbed_shape_errors(ext):
    x = torch.zeros(2, 1, 64)
    wa, g = torch.zeros(64, 32), torch.zeros(32)
    wb, wuk = torch.zeros(32, 4 * 24), torch.zeros(4, 16, 16)
    pos = torch.zeros(1, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="W_q_a must be"):
        ext.q_absorbed(x, wa[:60], g, wb, wuk, pos, 16, 8, 1e-6)
    with pytest.raises(RuntimeError, match="W_q_b must be"):
        ext.q_absorbed(x, wa, g, wb[:, :90], wuk, pos, 16, 8, 1e-6)
    with pytest.raises(RuntimeError, match="q_norm_w must be"):
        ext.q_absorbed(x, wa, g[:31], wb, wuk, pos, 16, 8, 1e-6)
    with pytest.raises(RuntimeError, match="positions must be"):
        ext.q_absorbed(x, wa, g, wb, wuk, torch.zeros(2, dtype=torch.int64), 16, 8, 1e-6)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        ext.q_absorbed(x, wa, g, wb, wuk, pos, 16, 8, 1e-6)


def test_binding_neighbour_shape_errors(ext):
    with pytest.raises(RuntimeError, match="nope_dim must lie"):
        ext.split_wkv_b(torch.zeros(2, 8, 16), 8)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        ext.split_wkv_b(torch.zeros(2, 8, 16), 4)
    x, W = torch.zeros(2, 1, 32), torch.zeros(32, 24)
    g, pos = torch.zeros(16), torch.zeros(1, dtype=torch.int64)
    ck, pe = torch.zeros(2, 5, 16), torch.zeros(2, 5, 8)
    with pytest.raises(RuntimeError, match="W_kv_a must be"):
        ext.kv_append(x, W[:, :20], g, pos, ck, pe, 0, 1e-6)
    with pytest.raises(RuntimeError, match="kv_norm_w must be"):
        ext.kv_append(x, W, g[:8], pos, ck, pe, 0, 1e-6)
    with pytest.raises(RuntimeError, match="must be contiguous"):
        ext.kv_append(x, W, g, pos, ck.transpose(1, 2).contiguous().transpose(1, 2), pe, 0, 1e-6)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        ext.kv_append(x, W, g, pos, ck, pe, 0, 1e-6)
    with pytest.raises(RuntimeError, match="W_o must be"):
        ext.o_proj(torch.zeros(2, 1, 4, 8), torch.zeros(30, 16))


def test_binding_paged_shape_errors(ext):
    qa, qr = torch.zeros(2, 1, 4, 16), torch.zeros(2, 1, 4, 8)
    ck, pe = torch.zeros(5, 64, 16), torch.zeros(5, 64, 8)
    tab, sl, wuv = torch.zeros(2, 2, dtype=torch.int32), torch.ones(2, dtype=torch.int32), torch.zeros(4, 8, 16)
    with pytest.raises(RuntimeError, match="block_table must be int32"):
        ext.mla_attention_paged(qa, qr, ck, pe, tab.long(), sl, wuv, 1.0)
    with pytest.raises(RuntimeError, match="seq_lens must be a 1-D"):
        ext.mla_attention_paged(qa, qr, ck, pe, tab, sl[:1], wuv, 1.0)
    with pytest.raises(RuntimeError, match="pe_pages must be"):
        ext.mla_attention_paged(qa, qr, ck, pe[:, :32], tab, sl, wuv, 1.0)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        ext.mla_attention_paged(qa, qr, ck, pe, tab, sl, wuv, 1.0)
    with pytest.raises(RuntimeError, match=r"positions must be \[B, Sq\]"):
        ext.kv_append_paged(torch.zeros(2, 1, 32), torch.zeros(32, 24), torch.zeros(16),
                            torch.zeros(1, dtype=torch.int64), tab, ck, pe, 1e-6)
    with pytest.raises(RuntimeError, match="positions must be"):
        ext.q_absorbed(torch.zeros(2, 1, 64), torch.zeros(64, 32), torch.zeros(32),
                       torch.zeros(32, 4 * 24), torch.zeros(4, 16, 16),
                       torch.zeros(3, 1, dtype=torch.int64), 16, 8, 1e-6)
    f8 = torch.zeros(5, 64, 16, dtype=torch.uint8), torch.zeros(5, 64, 8, dtype=torch.uint8)
    bf = lambda t: t.to(torch.bfloat16)  # noqa: E731
    with pytest.raises(RuntimeError, match="bfloat16 queries"):
        ext.mla_attention_paged_fp8kv(qa, qr, *f8, tab, sl, 1.0, wuv, 1.0)
    with pytest.raises(RuntimeError, match="float8_e4m3fn or uint8"):
        ext.mla_attention_paged_fp8kv(bf(qa), bf(qr), bf(ck), bf(pe), tab, sl, 1.0, bf(wuv), 1.0)
    with pytest.raises(RuntimeError, match="block_table must be int32"):
        ext.mla_attention_paged_fp8kv(bf(qa), bf(qr), *f8, tab.long(), sl, 1.0, bf(wuv), 1.0)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        ext.mla_attention_paged_fp8kv(bf(qa), bf(qr), *f8, tab, sl, 1.0, bf(wuv), 1.0)



def test_work_list_validation_and_size(lib):
    """The per-step view of the ragged work list: its length is wl_ints(B, max_items) and
    it is validated before any HIP call."""
    import wl_check as W
    for B, Sq, dt, bk in [(1, 1, F32, 16), (128, 1, BF16, 32), (300, 4, F32, 16)]:
        d = dsv3(B, Sq, 4992)
        rt = W.row_tiles_of(Sq, 128)
        n = lib.mla_attention_work_list_ints(dt, ctypes.byref(d))
        assert n == W.harness().wl_harness_ints(B, W.max_items(B, rt))
    d = dsv3(4, 1, 4992)
    n = lib.mla_attention_work_list_ints(F32, ctypes.byref(d))
    st = lib.mla_attention_work_list(F32, ctypes.byref(d), P16, P16, n - 1, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "ints" in _err(lib)
    st = lib.mla_attention_work_list(F32, ctypes.byref(d), None, P16, n, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "seq_lens" in _err(lib)
    d.batch = 0
    assert lib.mla_attention_work_list_ints(F32, ctypes.byref(d)) == 0
    st = lib.mla_attention_work_list(F32, ctypes.byref(d), P16, P16, n, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "batch" in _err(lib)


def test_noalloc_attention_validation(lib):
    """The allocation-free attention validates like mla_attention and rejects, before any HIP
    call, a shape whose workspace exceeds the library's fixed scratch (64 MiB per GPU)."""
    args = [P16] * 5
    limit = 64 << 20
    for B, Sq, Sk in [(128, 1, 4989), (1, 1, 65536), (64, 1, 4989), (8, 1, 4989)]:
        d = dsv3(B, Sq, Sk)
        for dt in (F32, BF16):
            assert lib.mla_attention_workspace_bytes(dt, ctypes.byref(d), 0) <= limit
    d = dsv3(4, 128, 32768)           # chunked prefill: 128 MiB of workspace
    assert lib.mla_attention_workspace_bytes(F32, ctypes.byref(d), 1) > limit
    st = lib.mla_attention_noalloc(F32, ctypes.byref(d), *args, ctypes.c_double(13.85), 1, P16,
                                   None)
    assert st == MLA_ERR_WORKSPACE and "scratch" in _err(lib)
    d = dsv3(2, 3, 2)
    st = lib.mla_attention_noalloc(F32, ctypes.byref(d), *args, ctypes.c_double(13.85), 1, P16,
                                   None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "sk >= sq" in _err(lib)
    d = dsv3(2, 1, 100)
    st = lib.mla_attention_noalloc(F32, ctypes.byref(d), P16, P16, None, P16, P16,
                                   ctypes.c_double(13.85), 0, P16, None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "c_kv" in _err(lib)
    st = lib.mla_attention_noalloc(F32, ctypes.byref(d), *args, ctypes.c_double(0.0), 0, P16,
                                   None)
    assert st == MLA_ERR_INVALID_ARGUMENT and "scale" in _err(lib)
