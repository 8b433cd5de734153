"""GPU test of mla_attention_noalloc, the allocation-free attention entry point.

It is called through the C ABI (ctypes on libmla_amd.so, device pointers of torch tensors,
torch's current stream) and compared with mla_attention, the entry point whose kernels it
shares, called through the C ABI with a caller workspace: bit for bit on two calls in a row
(the second with a smaller input, so it runs in scratch left over from the first), in fp32
and bf16, and against the CPU oracle.  A shape over the scratch limit is refused.  The first
test captures mla_attention_noalloc into a graph (torch.cuda.CUDAGraph); run first in a fresh
process, that capture holds the call's first use on the device, where the library looks up
the scratch array's address.
"""

from __future__ import annotations

import ctypes
import math
import os

import pytest
import torch

import attn_cases as C
from oracle import mla_ref as R

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "mla-cuda_amd", "libmla_amd.so")
DEV = "cuda:0"
D = R.DSV3
SCALE = math.sqrt(D.qk_head)
MLA_OK, MLA_ERR_WORKSPACE = 0, 3


class Dims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("batch", "sq", "sk", "hidden", "q_lora", "heads", "nope", "rope", "kv_rank", "v")]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    import mla_custom_cuda  # noqa: F401  (loads torch's HIP runtime and the library)
    L = ctypes.CDLL(LIB)
    L.mla_last_error.restype = ctypes.c_char_p
    L.mla_attention_workspace_bytes.restype = ctypes.c_size_t
    return L


def _inputs(B, Sq, Sk, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    s = 1 / math.sqrt(D.kv_rank)
    mk = lambda *shape, sc=1.0: (torch.randn(*shape, generator=g) * sc).to(dtype)  # noqa: E731
    return (mk(B, Sq, D.n_heads, D.kv_rank, sc=C.LAYER_QA_STD),
            mk(B, Sq, D.n_heads, D.rope, sc=C.LAYER_QR_STD),
            mk(B, Sk, D.kv_rank), mk(B, Sk, D.rope), mk(D.n_heads, D.v, D.kv_rank, sc=s))


def _call(lib, noalloc, dt, host, causal):
    qa, qr, ck, pe, wuv = [t.to(DEV) for t in host]
    B, Sq, H, Rk = qa.shape
    d = Dims(B, Sq, ck.shape[1], 7168, 1536, H, 128, qr.shape[3], Rk, wuv.shape[1])
    out = torch.empty(B, Sq, H, wuv.shape[1], dtype=qa.dtype, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptrs = [ctypes.c_void_p(t.data_ptr()) for t in (qa, qr, ck, pe, wuv)]
    if noalloc:
        st = lib.mla_attention_noalloc(dt, ctypes.byref(d), *ptrs, ctypes.c_double(SCALE),
                                       int(causal), ctypes.c_void_p(out.data_ptr()), stream)
    else:
        n = lib.mla_attention_workspace_bytes(dt, ctypes.byref(d), int(causal))
        ws = torch.empty(n, dtype=torch.uint8, device=DEV)
        st = lib.mla_attention(dt, ctypes.byref(d), *ptrs, ctypes.c_double(SCALE), int(causal),
                               ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                               ctypes.c_size_t(n), stream)
    assert st == MLA_OK, lib.mla_last_error().decode()
    torch.cuda.synchronize()
    return out.cpu()


def test_noalloc_under_graph_capture(lib):
    """mla_attention_noalloc captured into a graph (in a fresh process, its first call on the
    device, made inside the capture) and replayed four times with new inputs copied into
    the captured buffers; eager mla_attention and eager mla_attention_noalloc calls run
    between the replays, and every replay equals mla_attention bit for bit."""
    dtype, dt, B, Sq, Sk = torch.bfloat16, 1, 4, 1, 1000
    host = _inputs(B, Sq, Sk, seed=60, dtype=dtype)
    bufs = [t.to(DEV) for t in host]
    out = torch.empty(B, Sq, D.n_heads, D.v, dtype=dtype, device=DEV)
    d = Dims(B, Sq, Sk, 7168, 1536, D.n_heads, 128, D.rope, D.kv_rank, D.v)
    ptrs = [ctypes.c_void_p(t.data_ptr()) for t in bufs]
    torch.cuda.synchronize()
    print("noalloc graph capture: bf16 B=4 Sq=1 Sk=1000", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        st = lib.mla_attention_noalloc(dt, ctypes.byref(d), *ptrs, ctypes.c_double(SCALE), 0,
                                       ctypes.c_void_p(out.data_ptr()), stream)
    assert st == MLA_OK, lib.mla_last_error().decode()
    torch.cuda.synchronize()
    for i in range(4):
        h = host if i == 0 else _inputs(B, Sq, Sk, seed=60 + i, dtype=dtype)
        for buf, src in zip(bufs, h):
            buf.copy_(src.to(DEV))
        print(f"noalloc graph replay {i}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu()
        want = _call(lib, False, dt, h, False)
        assert torch.equal(got, want), f"replay {i} differs from mla_attention"
        assert torch.equal(_call(lib, True, dt, h, False), want)


@pytest.mark.parametrize("dtype,dt", [(torch.float32, 0), (torch.bfloat16, 1)],
                         ids=["f32", "bf16"])
def test_noalloc_matches_mla_attention(lib, dtype, dt):
    # the larger first: B=128 decode at the headline Sk; then B=3 (split keys, partials)
    for i, (B, Sq, Sk, causal) in enumerate([(128, 1, 4989, False), (3, 2, 700, True)]):
        print(f"noalloc {dtype} call {i}: B={B} Sq={Sq} Sk={Sk} causal={causal}", flush=True)
        host = _inputs(B, Sq, Sk, seed=40 + i, dtype=dtype)
        got = _call(lib, True, dt, host, causal)
        ref = _call(lib, False, dt, host, causal)
        assert torch.equal(got, ref), f"call {i} differs from mla_attention"
        if i == 1:
            f = [t.float() for t in host]
            oracle = R.mla_attention_official(*f, SCALE, causal=causal)
            torch.testing.assert_close(got.float(), oracle, **C.tol(dtype, oracle))


def test_noalloc_float64(lib):
    """float64 (MLA_DTYPE_F64) through the no-workspace entry point: two calls in a row, the
    second smaller, each bit for bit equal to mla_attention with a caller workspace."""
    for i, (B, Sq, Sk, causal) in enumerate([(2, 2, 1000, True), (1, 1, 300, False)]):
        print(f"noalloc float64 call {i}: B={B} Sq={Sq} Sk={Sk} causal={causal}", flush=True)
        host = _inputs(B, Sq, Sk, seed=70 + i, dtype=torch.float64)
        got = _call(lib, True, 3, host, causal)
        ref = _call(lib, False, 3, host, causal)
        assert got.dtype == torch.float64 and torch.equal(got, ref)


def test_noalloc_refuses_a_shape_over_its_scratch(lib):
    B, Sq, Sk = 4, 128, 1024          # 4*128*128 rows of ctx: 128 MiB of workspace
    d = Dims(B, Sq, Sk, 7168, 1536, D.n_heads, 128, D.rope, D.kv_rank, D.v)
    assert lib.mla_attention_workspace_bytes(0, ctypes.byref(d), 1) > (64 << 20)
    p = ctypes.c_void_p(1 << 20)
    st = lib.mla_attention_noalloc(0, ctypes.byref(d), p, p, p, p, p, ctypes.c_double(SCALE), 1,
                                   p, None)
    assert st == MLA_ERR_WORKSPACE and b"scratch" in lib.mla_last_error()
