#!/usr/bin/env python3
"""bench.py -- µs per absorbed-MLA layer on one MI355X, with per-step roofline figures.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2] [--no-cpu-baseline]

One "step" is one MLA layer, steps 2a1 -> 3d, through the drop-in surface
(mla_custom_cuda.q_absorbed + mla_custom_cuda.mla_attention), on inputs already resident
in HBM.  The default workload is the headline decode shape: B=128, Sq=1, Sk=4989, fp32,
DeepSeek-V3 dims.  Output: ONE JSON line on stdout.

Timed region: --settle seconds (default 2) of untimed layers, so the GPU clock has
reached the level it holds under sustained load, then W untimed warm-up layers, then
exactly K layers bracketed by
torch.cuda.synchronize() on both sides, each layer between its own pair of HIP events on
the current stream and preceded (outside the pair) by a 512 MB device read that evicts
the MALL and L2s (leaving clean lines); `value` is the mean per-layer time (median and a
back-to-back figure beside it).  A second, separately timed pass runs the same kernels through the per-step ops with an event
between consecutive steps; it gives each step's average launch duration, from which the
per-step GFLOP/s, GB/s, MFMA % and HBM % (algorithmic work, formulas below) and the
`roofline` object of the dominant kernel are computed.

With the default fp32 cfg2 workload the line also carries `bf16_cfg4`: the bf16 decode
(B=128, Sk=4989, bf16 storage) layer time and its fused attention's roofline, measured
the same way; and `other_configs`: every other BASELINE configuration in fp32 (cfg1 B=1
Sk=512; B=1, 8, 32 at Sk=4989; cfg5 B=4 Sq=128 Sk=32768 causal), each with its layer time,
in-layer kernel times, fused-attention roofline and the layer's roofline fraction (the sum
of the steps' bounds over the layer time).

cpu_baseline: the CPU oracle (oracle/mla_ref.py, the reference's PyTorch formulation
restated) timed on this machine's host cores on the same inputs -- the only place this
script touches oracle/.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "mla-cuda_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "µs per MLA layer (B=128 decode, Sk=4989) + HBM GB/s & MFMA util % per step"
PEAK_HBM = 8.0e12          # B/s, MI355X HBM3E
PEAK_F32 = 157.3e12        # flop/s, dense fp32 MFMA
PEAK_BF16 = 2.5e15         # flop/s, dense bf16 MFMA
REF_A6000_US = 16920.0     # reference's published layer time at this shape (README.md:367)

CONFIGS = {
    # name: (B, Sq, Sk, description)
    "cfg2": (128, 1, 4989, "B=128 Sq=1 Sk=4989 fp32 decode (headline workload)"),
    "cfg4": (128, 1, 4989, "B=128 Sq=1 Sk=4989 bf16 decode (bf16 storage, fp32 accumulation)"),
    "cfg1": (1, 1, 512, "B=1 Sq=1 Sk=512 fp32 decode (single short sequence)"),
    "b1": (1, 1, 4989, "B=1 Sq=1 Sk=4989 fp32 decode (small-batch sweep)"),
    "b8": (8, 1, 4989, "B=8 Sq=1 Sk=4989 fp32 decode (small-batch sweep)"),
    "b32": (32, 1, 4989, "B=32 Sq=1 Sk=4989 fp32 decode (small-batch sweep)"),
    "cfg5": (4, 128, 32768, "B=4 Sq=128 Sk=32768 fp32 causal chunked prefill (online-softmax attention)"),
}


# The reference's published scenario matrix (exhaustive_benchmark_suite.py:78-174; all
# non-causal, fp32) with its RTX A6000 figures in ms (README.md:366-375: PyTorch baseline,
# its fused CUDA path), and two prefill shapes it leaves out because their score matrix does
# not fit a 48 GB card (:75-76), run here unpublished.
#   name: (B, Sq, Sk, timed iterations, A6000 baseline ms, A6000 fused ms)
SCENARIOS = {
    "decode_single_user_long_ctx": (1, 1, 65536, 10, 1.91, 2.39),
    "decode_serving_avg_ctx": (128, 1, 4989, 15, 14.27, 16.92),
    "decode_serving_long_ctx": (128, 1, 8192, 15, 23.61, 26.55),
    "decode_serving_high_batch": (256, 1, 2048, 15, 12.91, 15.06),
    "decode_speculative_2tok": (64, 2, 512, 20, 2.59, 3.38),
    "decode_speculative_4tok": (64, 4, 768, 20, 6.16, 7.53),
    "decode_speculative_long_ctx": (132, 4, 4096, 10, 47.19, 54.90),
    "prefill_chat_batch": (8, 512, 512, 20, 70.55, 87.32),
    "prefill_chunk_2k": (1, 2048, 2048, 10, 94.15, 113.11),
    "prefill_chunk_4k": (1, 4096, 4096, 10, 355.46, 417.61),
    "prefill_chunk_8k": (1, 8192, 8192, 5, None, None),
    "prefill_batch_2k": (16, 2048, 2048, 5, None, None),
}


def torch_layer(g, W_uk, W_uv, dims, scale, eps=1e-6, causal=False):
    """The reference's PyTorch formulation of the layer (exhaustive_benchmark_suite.py:247-304:
    two projections around an RMSNorm, per-head absorption, interleaved RoPE, a softmax over
    the materialised scores) executed by torch on this GPU, its products on rocBLAS /
    hipBLASLt: the same-GPU library baseline.  In 16-bit the batched products get contiguous
    right operands (torch's batched 16-bit products have faulted on transposed views on this
    stack)."""
    import torch
    x = g["x"]
    B, Sq, _ = x.shape
    H, nope, rope, R = dims.n_heads, dims.nope, dims.rope, dims.kv_rank
    Sk = g["c_kv"].shape[1]
    lat = torch.matmul(x, g["W_q_a"]).float()
    lat = (lat * torch.rsqrt(lat.square().mean(-1, keepdim=True) + eps)).to(x.dtype) * g["q_norm_w"]
    q = torch.matmul(lat, g["W_q_b"]).view(B, Sq, H, nope + rope)
    q_nope = q[..., :nope].permute(2, 0, 1, 3).reshape(H, B * Sq, nope)
    qa = torch.bmm(q_nope, W_uk).view(H, B, Sq, R).permute(1, 2, 0, 3).reshape(B, Sq * H, R)
    inv = 1.0 / 10000 ** (torch.arange(0, rope, 2, device=x.device, dtype=torch.float32) / rope)
    ang = torch.outer(g["positions"].float(), inv)
    cos, sin = torch.cos(ang).view(1, Sq, 1, -1), torch.sin(ang).view(1, Sq, 1, -1)
    qp = q[..., nope:].float()
    ev, od = qp[..., 0::2], qp[..., 1::2]
    qr = torch.stack((ev * cos - od * sin, ev * sin + od * cos), -1).flatten(-2)
    qr = qr.to(x.dtype).reshape(B, Sq * H, rope)
    kT, pT, wT = g["c_kv"].transpose(1, 2), g["pe_cache"].transpose(1, 2), W_uv.transpose(1, 2)
    if x.dtype != torch.float32:
        kT, pT, wT = kT.contiguous(), pT.contiguous(), wT.contiguous()
    s = torch.bmm(qa, kT)
    s.add_(torch.bmm(qr, pT)).div_(scale)
    if causal:
        vis = (torch.arange(Sk, device=x.device)[None, :]
               <= torch.arange(Sk - Sq, Sk, device=x.device)[:, None])
        s.view(B, Sq, H, Sk).masked_fill_(~vis[None, :, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1)
    del s
    ctx = torch.bmm(p, g["c_kv"]).view(B, Sq, H, R).permute(2, 0, 1, 3).reshape(H, B * Sq, R)
    out = torch.bmm(ctx, wT)
    return out.view(H, B, Sq, -1).permute(1, 2, 0, 3)


def time_flushed(fn, iters, warmup, flush):
    """Mean ms of `iters` calls of fn, each preceded (outside its event pair) by a read of
    `flush` that evicts the MALL and L2s, after `warmup` calls made the same way."""
    import torch
    for _ in range(warmup):
        flush.sum()
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(iters)]
    for e0, e1 in ev:
        flush.sum()
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return statistics.mean(e0.elapsed_time(e1) for e0, e1 in ev)


def graph_vs_eager(layer, out_ref, n, settle_s, marker=None):
    """Capture `layer` in a HIP graph, replay it for `settle_s` seconds (the capture leaves the
    GPU idle, and the clock dips for ~100 ms after an idle spell before it settles), check the
    replay against `out_ref` bit for bit, then time two rounds of n eager layers back to back
    followed by n replays; returns (eager µs, replay µs) per layer of the last round.
    `marker`, a small device tensor, gets an in-place op before each timed region so a kernel
    trace shows where each region starts."""
    import torch
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = layer()
    t0 = time.perf_counter()
    while True:
        for _ in range(10):
            graph.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= settle_s:
            break
    if not torch.equal(out_g, out_ref):
        raise RuntimeError("graph replay differs from the eager layer")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for _ in range(2):
        if marker is not None:
            marker.add_(1.0)
        ev[0].record()
        for _ in range(n):
            layer()
        ev[1].record()
        if marker is not None:
            marker.mul_(2.0)
        ev[2].record()
        for _ in range(n):
            graph.replay()
        ev[3].record()
        torch.cuda.synchronize()
    del graph, out_g
    return ev[0].elapsed_time(ev[1]) / n * 1e3, ev[2].elapsed_time(ev[3]) / n * 1e3


def in_layer_kernel_us(layer, flush, n):
    """Each step's kernel time inside the real layer: n flush-then-layer iterations under
    torch's profiler (kernel start and end from the GPU's own timestamps), the library's
    kernels attributed to steps by launch order -- the layer launches its GEMMs in the order
    2a1, 2a2, 2c, 3d, a split-K reduce right after its GEMM, RMSNorm (2a-n, which also sums
    2a1's split partials) and RoPE (2b) between them (the 16-bit 2a2 may do 2b and 2c in its
    epilogue: `wgemm_kernel<.., 2, false>`, counted as 2a2; an unsplit fp32 2a2 may do 2b:
    `gemm_kernel<.., true>`, its last template argument; at decode-sized fp32 batches
    `q_small_kernel` does 2b and 2c, counted as 2c), and the fused attention's kernels
    (work list, pass, merge) as 3abc; at decode-sized fp32 batches 3d may be
    out_small_kernel, which also does the pass's split merge.  Returns {step: mean µs per
    layer} plus the layer's
    span from its first kernel's start to its last kernel's end, or None if the profiler
    records no kernels."""
    import torch
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(n):
            flush.sum()
            layer()
        torch.cuda.synchronize()
    ks = []
    for e in prof.events():
        if e.device_type != torch.autograd.DeviceType.CUDA:
            continue
        ks.append((e.time_range.start, e.time_range.end, e.name))
    return attribute_steps(ks)


# the fused path's steps, in launch order
FUSED_PATH = ("2a1", "2a-n", "2a2", "2b", "2c", "3abc", "3d")


def attribute_steps(ks):
    """`in_layer_kernel_us`'s attribution of kernel records (start, end, demangled name) to
    steps, as described there; records of other kernels (the flush) separate the layers."""
    ks = sorted(ks)
    gemm_steps = ("2a1", "2a2", "2c", "3d")
    folded = {}                       # step -> the steps its kernel also does
    tot = {}
    spans = []
    layers = 0
    cur = None
    for t0, t1, name in ks:
        if not any(k in name for k in ("gemm_kernel", "split_reduce", "rmsnorm_kernel",
                                        "rope_kernel", "q_small", "flash", "out_small")):
            cur = None                # the flush between layers
            continue
        if cur is None:
            cur = {"gemm": 0, "step": None, "t0": t0}
            layers += 1
            spans.append([t0, t1])
        spans[-1][1] = t1
        if "gemm_kernel" in name:
            step = gemm_steps[min(cur["gemm"], 3)]
            cur["gemm"] += 1
            if "wgemm_kernel" in name and re.search(r",\s*2(,\s*(false|true))?>", name):
                cur["gemm"] += 1      # 2a2 with 2b and 2c in its epilogue: no 2c launch
                folded["2a2"] = ("2b", "2c")
            elif step == "2a2" and "wgemm_kernel" not in name and re.search(r",\s*true>", name):
                folded["2a2"] = ("2b",)   # the fp32 2a2 that rotates q_rope in its epilogue
        elif "split_reduce" in name:
            step = cur["step"] or "2a1"
        elif "rmsnorm" in name:
            step = "2a-n"
        elif "rope_kernel" in name:
            step = "2b"
        elif "q_small" in name:       # 2b and 2c in one kernel at decode-sized fp32 batches
            step = "2c"
            cur["gemm"] += 1
            folded["2c"] = ("2b",)
        elif "flash" in name:
            step = "3abc"
        elif "out_small" in name:      # 3d with the attention's split merge folded in
            step = "3d"
        else:
            step = "other"
        cur["step"] = step
        tot[step] = tot.get(step, 0.0) + (t1 - t0)
    if not layers:
        return None
    # another profiler attached to the process (rocprofv3) leaves torch's kernel records
    # with durations of ~1 us; such a reading is no measurement
    if sum(tot.values()) < 0.5 * sum(b - a for a, b in spans):
        return None
    out = {k: round(v / layers, 2) for k, v in tot.items()}
    out["kernels_sum"] = round(sum(tot.values()) / layers, 2)
    out["layer_span"] = round(sum(b - a for a, b in spans) / layers, 2)
    out["layers"] = layers
    out["folded"] = folded
    return out


def step_work(B, Sq, Sk, dims, e=4, causal=False):
    """Algorithmic FLOPs and compulsory HBM bytes per step (each input read once, each
    output written once; fp32 intermediates).  FLOP formulas follow the reference's own
    roofline (stage_profile.py:85-93); with a causal mask the score and ctx FLOPs count the
    keys a query sees, Sk - Sq + 1 + i for query i, i.e. Sk - (Sq - 1) / 2 on average."""
    H, R, D, V = dims.n_heads, dims.kv_rank, dims.rope, dims.v
    hid, ql, qk, nope = dims.hidden, dims.q_lora, dims.qk_head, dims.nope
    bq = B * Sq
    flat = bq * H
    P = -(-Sk // 128)
    Sv = Sk - (Sq - 1) / 2 if causal else Sk     # mean visible keys per query
    w = {
        "2a1": (2 * bq * hid * ql, e * (bq * hid + hid * ql) + 4 * bq * ql),
        "2a-n": (3 * bq * ql, 4 * bq * ql + e * ql + e * bq * ql),
        "2a2": (2 * bq * ql * H * qk, e * (bq * ql + ql * H * qk) + 4 * bq * H * qk),
        "2b": (6 * bq * H * D // 2, 4 * bq * H * D + e * bq * H * D),
        "2c": (2 * bq * H * nope * R, 4 * bq * H * nope + e * H * nope * R + e * bq * H * R),
        "3a": (2 * flat * Sv * (R + D), e * (flat * (R + D) + B * Sk * (R + D))
               + 4 * (flat * Sk + 2 * flat * P)),
        "3b": (3 * flat * P, 4 * (3 * flat * P + flat)),
        "3c": (2 * flat * Sv * R, 4 * (flat * Sk + flat * P) + e * (B * Sk * R) + 4 * flat * R),
        "3d": (2 * flat * R * V, 4 * flat * R + e * H * V * R + 4 * flat + e * flat * V),
        # 3a+3b+3c fused (the layer's attention kernel at kv_rank 512 / rope 64): queries
        # and cache read once, the unnormalised ctx and row sums written once
        "3abc": (2 * flat * Sv * (R + D) + 2 * flat * Sv * R,
                 e * (flat * (R + D) + B * Sk * (R + D)) + 4 * flat * R + 4 * flat),
    }
    return w


def build_inputs(B, Sq, Sk, seed=0, dtype=None):
    import torch
    import mla_inputs
    return mla_inputs.make_inputs(B, Sq, Sk, seed=seed, dtype=dtype or torch.float32)


def cpu_baseline(inp, gpu_out, budget_s=30.0, causal=False):
    """Time the CPU oracle on the host cores: 1 warm-up, then the median of up to 3 runs,
    on the full workload if one layer fits the budget, else on the first sequences of the
    batch (scaled to the full batch; every sequence costs the same)."""
    import torch
    from oracle import mla_ref as R

    threads = max(1, min(16, os.cpu_count() or 1))
    torch.set_num_threads(threads)
    B = inp["x"].shape[0]

    inp = {k: (v.float() if v.is_floating_point() else v) for k, v in inp.items()}

    def layer(b):
        return R.mla_layer(inp["x"][:b], inp["W_q_a"], inp["q_norm_w"], inp["W_q_b"],
                           inp["wkv_b"], inp["c_kv"][:b], inp["pe_cache"][:b],
                           inp["positions"], causal=causal)

    # probe with a small sample to size the run
    bs = min(B, 8)
    t0 = time.perf_counter()
    ref = layer(bs)
    t_probe = time.perf_counter() - t0
    est_full = t_probe * B / bs
    b_use = B if est_full * 4 <= budget_s else max(1, min(B, int(budget_s / 4 / (t_probe / bs))))
    ref = layer(b_use)  # warm-up at the chosen size
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        ref = layer(b_use)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    us = t * 1e6 * (B / b_use)
    err = (gpu_out[:b_use].float().cpu() - ref).abs().max().item()
    sample = (f"{'full batch' if b_use == B else f'first {b_use} of {B} sequences, scaled x{B / b_use:.1f}'}"
              f"; oracle layer on CPU, 1 warm-up + median of 3")
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f
                          if ln.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(us, 1), "unit": "µs", "cores": threads, "kind": "port",
            "sample": sample, "torch_threads": torch.get_num_threads(),
            "os_cpu_count": os.cpu_count(), "cpu_model": model}, err, b_use


def measure(args, ext, dev, neighbours=True, light=False):
    """Time one configuration (args.config, args.dtype); returns the JSON record.
    light: only the layer (flushed and back to back), its in-layer kernel times and the
    fused attention's own timing -- no torch formulation, graph replay or per-step pass."""
    import torch
    import mla_inputs

    dims = mla_inputs.DEEPSEEK_V3
    B, Sq, Sk, desc = CONFIGS[args.config]
    dname = args.dtype or ("bf16" if args.config == "cfg4" else "f32")
    dt = {"bf16": torch.bfloat16, "f16": torch.float16}.get(dname, torch.float32)
    half = dname != "f32"   # 16-bit storage and MFMA (bf16 or fp16)
    if half and dname not in desc:
        desc = desc.replace("fp32", dname).replace("bf16", dname)
    print(f"[bench] config {args.config}: {desc}", file=sys.stderr, flush=True)

    inp = build_inputs(B, Sq, Sk, args.seed, dt)
    W_uk = inp["wkv_b"][:, :dims.nope, :].contiguous()
    W_uv = inp["wkv_b"][:, dims.nope:, :].contiguous()
    g = {k: v.to(dev) for k, v in inp.items()}
    W_uk_d, W_uv_d = W_uk.to(dev), W_uv.to(dev)
    scale = math.sqrt(dims.qk_head)
    eps = 1e-6

    causal = args.config == "cfg5"
    fp8kv = args.kv_cache == "fp8"
    if fp8kv:
        # the layer's cache as fp8 e4m3 codes with one per-tensor scale (amax / 448); the
        # per-step pass and the neighbours below keep the bf16 cache
        if dname != "bf16":
            raise SystemExit("--kv-cache fp8 needs bf16 queries (--dtype bf16 or cfg4)")
        kv_scale = float(torch.maximum(g["c_kv"].abs().max(), g["pe_cache"].abs().max()).float()) / 448.0
        ck_l = (g["c_kv"].float() / kv_scale).to(torch.float8_e4m3fn)
        pe_l = (g["pe_cache"].float() / kv_scale).to(torch.float8_e4m3fn)

    def layer():
        qa, qr = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"], W_uk_d,
                                g["positions"], dims.nope, dims.rope, eps)
        if fp8kv:
            return ext.mla_attention_fp8kv(qa, qr, ck_l, pe_l, kv_scale, W_uv_d, scale, causal)
        # causal (cfg5) too: the fused pass streams the keys through its online softmax
        # and keeps no score matrix
        return ext.mla_attention(qa, qr, g["c_kv"], g["pe_cache"], W_uv_d, scale, causal)

    if args.graph_compare:
        # only the graph-versus-eager comparison, 50 layers a region, with marker kernels
        # between the regions for a kernel trace
        out = layer()
        torch.cuda.synchronize()
        marker = torch.zeros(3, device=dev)
        eager_us, graph_us = graph_vs_eager(layer, out, 50, args.settle, marker)
        print(f"[bench] eager back to back {eager_us:.1f} µs/layer, graph replay "
              f"{graph_us:.1f} µs/layer", file=sys.stderr, flush=True)
        return {"graph_compare": args.config, "dtype": dname, "layers_per_region": 50,
                "eager_b2b_us_per_step": round(eager_us, 2),
                "graph_replay_us_per_step": round(graph_us, 2),
                "config": {"workload": desc, "B": B, "Sq": Sq, "Sk": Sk}}

    # ---- timed region: the fused boundary calls.  Each timed layer is preceded by a 512 MB
    # device read outside its event pair, so no layer finds the previous one's weights or
    # cache in the 256 MB MALL or the L2s; value = mean over the layers (median beside it).
    # The flush reads rather than writes: a write leaves ~256 MB of dirty lines whose
    # write-back then competes with the timed layer's own reads (measured: the B=1 q
    # up-projection's 151 MB weight stream takes 53 us after a write flush, 34 us after a
    # read), a cost a decode loop, whose big traffic is weight and cache reads, does not pay.
    # The warm-up layers follow the same flush-then-layer pattern.
    # The GPU's clock follows the load over seconds: after an idle spell the first few
    # milliseconds run fast, the next ~100 ms dip 20-35% below the level the clock holds
    # after ~2 s of sustained work (measured on the fused bf16 attention, back to back:
    # ~215 us per call, then 290-337 us, then 215-225 us from about 2 s on).  A serving
    # loop runs at that settled level, so --settle seconds (default 2) of the same
    # flush-then-layer loop precede the warm-up layers.
    flush = torch.zeros(512 << 18, dtype=torch.float32, device=dev)   # 512 MB
    t_settle = time.perf_counter()
    n_settle = 0
    while time.perf_counter() - t_settle < args.settle:
        for _ in range(10):
            flush_sum = flush.sum()   # noqa: F841
            out = layer()
        torch.cuda.synchronize()
        n_settle += 10
    for _ in range(args.warmup):
        flush_sum = flush.sum()   # noqa: F841
        out = layer()
    torch.cuda.synchronize()
    lev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    t_wall = time.perf_counter()
    for e0, e1 in lev:
        flush_sum = flush.sum()   # noqa: F841  (reads all 512 MB)
        e0.record()
        out = layer()
        e1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    layer_ms = [e0.elapsed_time(e1) for e0, e1 in lev]
    ms_per_step = statistics.mean(layer_ms)
    ms_median = statistics.median(layer_ms)
    print(f"[bench] fused layer, eager launches, flushed caches: mean {ms_per_step * 1e3:.1f} "
          f"µs, median {ms_median * 1e3:.1f} µs over {args.steps} layers", file=sys.stderr,
          flush=True)
    # the same calls back to back (caches warm from the previous layer)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        out = layer()
    end.record()
    torch.cuda.synchronize()
    b2b_us = round(start.elapsed_time(end) / args.steps * 1e3, 2)

    # each step's kernel time inside the flushed layer (GPU timestamps, no events between
    # the steps), for the fused path
    in_layer = None
    if os.environ.get("MLA_ATTENTION_PATH") != "split":
        try:
            in_layer = in_layer_kernel_us(layer, flush, min(10, args.steps))
        except Exception as e:   # the profiler is a measurement aid, not the product
            print(f"[bench] in-layer kernel times unavailable ({e})", file=sys.stderr, flush=True)
        if in_layer:
            print("[bench] in-layer kernel µs: " + ", ".join(f"{k} {v}" for k, v in in_layer.items()),
                  file=sys.stderr, flush=True)

    # the same layer through torch on this GPU (the reference's PyTorch formulation,
    # rocBLAS / hipBLASLt products), timed with the same flush-then-layer protocol
    torch_same = None
    if not fp8kv and not light:
        try:
            def t_layer():
                return torch_layer(g, W_uk_d, W_uv_d, dims, scale, eps, causal)
            t_out = t_layer()
            t_diff = (t_out.float() - out.float()).abs().max().item()
            del t_out
            t_ms = time_flushed(t_layer, args.steps, min(5, args.warmup), flush)
            torch_same = {"us": round(t_ms * 1e3, 2),
                          "torch_over_layer": round(t_ms / ms_per_step, 3),
                          "max_abs_diff_vs_layer": t_diff}
            print(f"[bench] torch formulation on this GPU: {t_ms * 1e3:.1f} µs "
                  f"({t_ms / ms_per_step:.2f}x the layer)", file=sys.stderr, flush=True)
        except torch.cuda.OutOfMemoryError:
            torch_same = {"us": None, "note": "out of memory"}
        torch.cuda.empty_cache()
    del flush

    # The same layer replayed from a HIP graph (captured once; every replay runs all of the
    # layer's kernels), as a serving loop would launch it, against eager launches back to
    # back, both after the replays have settled the clock again.  The replay must reproduce
    # the eager output bit for bit.
    graph_us = b2b_settled_us = None
    try:
        if not light:
            b2b_settled_us, graph_us = graph_vs_eager(layer, out, args.steps, args.settle)
            print(f"[bench] fused layer, graph replay: {graph_us:.1f} µs/step (eager back to "
                  f"back {b2b_settled_us:.1f})", file=sys.stderr, flush=True)
    except RuntimeError as e:
        print(f"[bench] graph replay unavailable ({e})", file=sys.stderr, flush=True)

    # ---- per-step pass: same kernels via the per-step ops, an event between steps
    x2d = g["x"].reshape(B * Sq, dims.hidden)
    names = ["2a1", "2a-n", "2a2", "2b", "2c", "3a", "3b", "3c", "3d"]

    def steps(ev):
        ev[0].record()
        lat_acc = ext.gemm(x2d, g["W_q_a"]); ev[1].record()
        lat = ext.rmsnorm(lat_acc, g["q_norm_w"], eps); ev[2].record()
        raw = ext.gemm(lat, g["W_q_b"]); ev[3].record()
        qr = ext.rope(raw, g["positions"], B, Sq, dims.n_heads, dims.nope, dims.rope,
                      dt); ev[4].record()
        qa = ext.absorb(raw, W_uk_d, B, Sq, dims.rope); ev[5].record()
        p, m, l = ext.scores(qa, qr, g["c_kv"], g["pe_cache"], scale, causal); ev[6].record()
        alpha, rs = ext.combine(m, l); ev[7].record()
        ctx = ext.ctx(p, alpha, g["c_kv"], Sq, dims.n_heads); ev[8].record()
        o = ext.out(ctx, rs, W_uv_d); ev[9].record()
        return o

    if light:
        names, step_us, steps_sum, same = [], {}, None, None
    else:
        for _ in range(2):
            steps([torch.cuda.Event(enable_timing=True) for _ in range(10)])
        torch.cuda.synchronize()
        all_ev = [[torch.cuda.Event(enable_timing=True) for _ in range(10)]
                  for _ in range(args.steps)]
        for ev in all_ev:
            o_steps = steps(ev)
        torch.cuda.synchronize()
        step_us = {n: statistics.mean(ev[i].elapsed_time(ev[i + 1]) for ev in all_ev) * 1e3
                   for i, n in enumerate(names)}
        steps_sum = sum(step_us.values())
        same = (o_steps - out).abs().max().item()

    # the layer's attention runs 3a+3b+3c as one fused kernel (attn_ctx) at the
    # DeepSeek-V3 widths, timed here the same way; the per-step 3a/3b/3c above are the
    # decomposed kernels
    fused_attn = (dims.kv_rank == 512 and dims.rope == 64
                  and os.environ.get("MLA_ATTENTION_PATH") != "split")
    if fused_attn and fp8kv:
        # the fp8-cache pass has no entry point of its own: its time is the in-layer kernel
        # time of the layer's pass (GPU timestamps), when the profiler gave one
        if in_layer and "3abc" in in_layer:
            step_us["3abc"] = in_layer["3abc"]
            names = names + ["3abc"]
    elif fused_attn:
        qa_f, qr_f = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"], W_uk_d,
                                    g["positions"], dims.nope, dims.rope, eps)
        for _ in range(2):
            ext.attn_ctx(qa_f, qr_f, g["c_kv"], g["pe_cache"], scale, causal)
        torch.cuda.synchronize()
        fev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        for e0, e1 in fev:
            e0.record()
            ext.attn_ctx(qa_f, qr_f, g["c_kv"], g["pe_cache"], scale, causal)
            e1.record()
        torch.cuda.synchronize()
        step_us["3abc"] = statistics.mean(e0.elapsed_time(e1) for e0, e1 in fev) * 1e3
        names = names + ["3abc"]

    work = step_work(B, Sq, Sk, dims, e=2 if half else 4, causal=causal)
    if fp8kv:
        # the fp8-cache pass: bf16 queries, one byte per cache element, the normalised bf16
        # ctx written once (3d reads it)
        flat = B * Sq * dims.n_heads
        width = dims.kv_rank + dims.rope
        work["3abc"] = (work["3abc"][0],
                        2 * flat * width + B * Sk * width + 2 * flat * dims.kv_rank)
    peak_mfma = PEAK_BF16 if half else PEAK_F32   # the fp16 MFMA peak equals the bf16 one
    per_step = {}
    for n in names:
        fl, by = work[n]
        t = step_us[n] * 1e-6
        per_step[n] = {"us": round(step_us[n], 2), "gflop": round(fl / 1e9, 3),
                       "mbytes": round(by / 1e6, 2),
                       "tflops": round(fl / t / 1e12, 2), "gbps": round(by / t / 1e9, 1),
                       "mfma_pct": round(100 * fl / t / peak_mfma, 1),
                       "hbm_pct": round(100 * by / t / PEAK_HBM, 1)}
    dom = "3abc" if fused_attn else max(("3a", "3c"), key=lambda n: step_us[n])
    fl, by = work[dom]
    t_dom = step_us[dom] * 1e-6 if dom in step_us else None
    if t_dom is None:
        roofline = {"kernel": dom, "bound": None, "achieved": None, "peak": None,
                    "unit": None, "frac": None}
    elif fl / by > peak_mfma / PEAK_HBM:   # above the ridge: compute-bound
        achieved = fl / t_dom / 1e12
        roofline = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2),
                    "peak": peak_mfma / 1e12, "unit": "TFLOP/s",
                    "frac": round(achieved / (peak_mfma / 1e12), 4)}
    else:
        achieved = by / t_dom / 1e9
        roofline = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1),
                    "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                    "frac": round(achieved / (PEAK_HBM / 1e9), 4)}
    traffic = None
    try:
        with open(args.traffic) as f:
            tr = json.load(f)
        key = f"{args.config}/{dname}{'-fp8kv' if fp8kv else ''}/{dom}"
        if key in tr.get("kernels", {}):
            traffic = tr["kernels"][key]["hbm_bytes_per_launch"]
    except (OSError, ValueError):
        traffic = None
    roofline.update({"traffic": traffic, "algorithmic_flop": fl, "algorithmic_bytes": by})
    if fp8kv:
        roofline["timing"] = "the pass's kernel time inside the layer (GPU timestamps)"

    in_layer_steps = None
    fused_steps = ("2a1", "2a-n", "2a2", "2b", "2c", "3abc", "3d")
    if in_layer:
        # each kernel's duration inside the flushed layer as the profiler measured it; the
        # figures are reported as measured.  The profiler's session runs the kernels a few
        # to ~15% longer than the event-timed layers, so `layer_over_span` (event-timed
        # layer / profiled span, <= 1) is given beside them for reference only.
        span_il = in_layer["layer_span"]
        in_layer_steps = {"layer_over_span": (round(min(1.0, ms_per_step * 1e3 / span_il), 4)
                                              if span_il > 0 else None)}
        for n in fused_steps:
            if n not in in_layer:
                continue
            fl, by = work[n]
            for f in in_layer.get("folded", {}).get(n, ()):   # steps its kernel also does
                fl, by = fl + work[f][0], by + work[f][1]
            t = in_layer[n] * 1e-6
            in_layer_steps[n] = {"us": in_layer[n],
                                 "tflops": round(fl / t / 1e12, 2),
                                 "gbps": round(by / t / 1e9, 1),
                                 "mfma_pct": round(100 * fl / t / peak_mfma, 1),
                                 "hbm_pct": round(100 * by / t / PEAK_HBM, 1)}
        in_layer_steps["kernels_sum_us"] = in_layer["kernels_sum"]
        in_layer_steps["layer_span_us"] = in_layer["layer_span"]

    # the layer against its roofline: the sum over the fused path's steps of each step's
    # bound max(FLOPs / MFMA peak, bytes / HBM peak), and the in-layer kernel that takes
    # the most time with its own roofline fraction
    def bound_us(n):
        fl_n, by_n = work[n]
        return max(fl_n / peak_mfma, by_n / PEAK_HBM) * 1e6
    layer_bound_us = sum(bound_us(n) for n in fused_steps)
    dominant_in_layer = None
    if in_layer_steps:
        cand = [n for n in fused_steps if n in in_layer_steps]
        top = max(cand, key=lambda n: in_layer_steps[n]["us"])
        fl_t, by_t = work[top]
        t = in_layer_steps[top]["us"] * 1e-6
        mf = fl_t / by_t > peak_mfma / PEAK_HBM
        ach = fl_t / t / 1e12 if mf else by_t / t / 1e9
        pk = peak_mfma / 1e12 if mf else PEAK_HBM / 1e9
        dominant_in_layer = {"kernel": top, "us": in_layer_steps[top]["us"],
                             "bound": "mfma" if mf else "hbm", "achieved": round(ach, 2),
                             "peak": pk, "unit": "TFLOP/s" if mf else "GB/s",
                             "frac": round(ach / pk, 4)}

    nb = {}
    if neighbours:
        # ---- the path's neighbours, timed separately (not part of the layer's value):
        # the wkv_b split (weight prep), the KV-cache append of this step's Sq tokens per
        # sequence, and the output projection wo of the layer's output.
        e_b = 2 if half else 4
        H, R_, D_, V_, hid = dims.n_heads, dims.kv_rank, dims.rope, dims.v, dims.hidden
        bq = B * Sq
        gen = torch.Generator(device=dev).manual_seed(args.seed + 1)
        W_kv_a = (torch.randn(hid, R_ + D_, device=dev, generator=gen) / math.sqrt(hid)).to(dt)
        kv_gain = (1.0 + 0.1 * torch.randn(R_, device=dev, generator=gen)).to(dt)
        W_o = (torch.randn(H * V_, hid, device=dev, generator=gen) / math.sqrt(H * V_)).to(dt)
        kv_pos = torch.arange(Sk - Sq, Sk, device=dev)
        nb_calls = {
            "split_wkv_b": (lambda: ext.split_wkv_b(g["wkv_b"], dims.nope),
                            0, 2 * e_b * H * (dims.nope + V_) * R_),
            "kv_append": (lambda: ext.kv_append(g["x"], W_kv_a, kv_gain, kv_pos, g["c_kv"],
                                                g["pe_cache"], Sk - Sq, eps),
                          2 * bq * hid * (R_ + D_),
                          e_b * (bq * hid + hid * (R_ + D_) + R_ + bq * (R_ + D_)) + 8 * Sq),
            "o_proj": (lambda: ext.o_proj(out, W_o), 2 * bq * H * V_ * hid,
                       e_b * (bq * H * V_ + H * V_ * hid + bq * hid)),
        }
        for name, (fn, fl, by) in nb_calls.items():
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) / args.steps * 1e-3
            mfma_bound = fl > 0 and fl / by > peak_mfma / PEAK_HBM
            frac = (fl / t / peak_mfma) if mfma_bound else (by / t / PEAK_HBM)
            nb[name] = {"us": round(t * 1e6, 2), "gflop": round(fl / 1e9, 3),
                        "mbytes": round(by / 1e6, 2), "tflops": round(fl / t / 1e12, 2),
                        "gbps": round(by / t / 1e9, 1), "bound": "mfma" if mfma_bound else "hbm",
                        "frac": round(frac, 4)}
        # attention alone over the same keys: dense, then through a shuffled pool of 64-key
        # pages (full lengths: the dense work, plus the page-table indirection), then with
        # ragged lengths U[1, Sk] (work is still that of the longest sequence: masked tiles
        # are computed)
        if not causal:
            page = 64
            mp = -(-Sk // page)
            gp = torch.Generator().manual_seed(args.seed + 2)
            perm = torch.randperm(B * mp, generator=gp)
            pad = mp * page - Sk
            def pool(t):
                tp = torch.nn.functional.pad(t, (0, 0, 0, pad)).reshape(B * mp, page, t.shape[-1])
                out_pool = torch.empty_like(tp)
                out_pool[perm.to(dev)] = tp
                return out_pool
            ck_pool, pe_pool = pool(g["c_kv"]), pool(g["pe_cache"])
            table = perm.reshape(B, mp).int().to(dev)
            full = torch.full((B,), Sk, dtype=torch.int32, device=dev)
            ragged = torch.randint(1, Sk + 1, (B,), generator=gp, dtype=torch.int32).to(dev)
            qa_b, qr_b = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"], W_uk_d,
                                        g["positions"], dims.nope, dims.rope, eps)
            fl_attn = work["3a"][0] + work["3c"][0] + work["3d"][0]
            keys_ragged = int(ragged.sum().item())
            att_calls = {
                "attention_dense": (lambda: ext.mla_attention(qa_b, qr_b, g["c_kv"], g["pe_cache"],
                                                              W_uv_d, scale), fl_attn),
                "attention_paged": (lambda: ext.mla_attention_paged(
                    qa_b, qr_b, ck_pool, pe_pool, table, full, W_uv_d, scale), fl_attn),
                "attention_paged_ragged": (lambda: ext.mla_attention_paged(
                    qa_b, qr_b, ck_pool, pe_pool, table, ragged, W_uv_d, scale),
                    fl_attn * keys_ragged / (B * Sk)),
            }
            if dname == "bf16":
                # the same attention over an fp8 (e4m3) copy of the cache, one per-tensor
                # scale (amax / 448): half the cache bytes
                kv_scale = float(torch.maximum(g["c_kv"].abs().max(),
                                               g["pe_cache"].abs().max()).float()) / 448.0
                ck8 = (g["c_kv"].float() / kv_scale).to(torch.float8_e4m3fn)
                pe8 = (g["pe_cache"].float() / kv_scale).to(torch.float8_e4m3fn)
                att_calls["attention_fp8kv"] = (lambda: ext.mla_attention_fp8kv(
                    qa_b, qr_b, ck8, pe8, kv_scale, W_uv_d, scale), fl_attn)
                # and over the same pages as fp8 codes, at the ragged lengths
                ck8_pool = (ck_pool.float() / kv_scale).to(torch.float8_e4m3fn)
                pe8_pool = (pe_pool.float() / kv_scale).to(torch.float8_e4m3fn)
                att_calls["attention_paged_ragged_fp8kv"] = (lambda: ext.mla_attention_paged_fp8kv(
                    qa_b, qr_b, ck8_pool, pe8_pool, table, ragged, kv_scale, W_uv_d, scale),
                    fl_attn * keys_ragged / (B * Sk))
            for name, (fn, fl) in att_calls.items():
                for _ in range(3):
                    fn()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(args.steps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                t = e0.elapsed_time(e1) / args.steps * 1e-3
                nb[name] = {"us": round(t * 1e6, 2), "gflop": round(fl / 1e9, 3),
                            "tflops": round(fl / t / 1e12, 2), "bound": "mfma" if dname == "f32" else "hbm",
                            "mfma_pct": round(100 * fl / t / peak_mfma, 1)}
            nb["attention_paged_ragged"]["mean_keys"] = round(keys_ragged / B, 1)
            if "attention_fp8kv" in nb:
                nb["attention_fp8kv"]["cache_mbytes"] = round(B * Sk * (dims.kv_rank + dims.rope) / 1e6, 1)
                nb["attention_paged_ragged_fp8kv"]["mean_keys"] = round(keys_ragged / B, 1)
                del ck8, pe8, ck8_pool, pe8_pool
            del ck_pool, pe_pool
        else:
            # causal: the key-chunked entry point (bounded score workspace) beside the layer's
            # fused pass
            qa_b, qr_b = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"], W_uk_d,
                                        g["positions"], dims.nope, dims.rope, eps)
            fl_attn = work["3a"][0] + work["3c"][0] + work["3d"][0]
            fn = lambda: ext.mla_attention_streaming(qa_b, qr_b, g["c_kv"], g["pe_cache"],  # noqa: E731
                                                     W_uv_d, scale, True)
            fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) / args.steps * 1e-3
            nb["attention_streaming_chunks"] = {
                "us": round(t * 1e6, 2), "gflop": round(fl_attn / 1e9, 3),
                "tflops": round(fl_attn / t / 1e12, 2), "bound": "mfma",
                "mfma_pct": round(100 * fl_attn / t / peak_mfma, 1)}
        print(f"[bench] neighbours: " + ", ".join(f"{k} {v['us']} µs" for k, v in nb.items()),
              file=sys.stderr, flush=True)

    value_us = ms_per_step * 1e3
    rec = {
        "metric": METRIC,
        "value": round(value_us, 2),
        "unit": "µs",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": args.settle,
        "settle_layers": n_settle,
        "ms_per_step": round(ms_per_step, 4),
        "median_us_per_step": round(ms_median * 1e3, 2),
        "min_max_us_per_step": [round(min(layer_ms) * 1e3, 2), round(max(layer_ms) * 1e3, 2)],
        "back_to_back_us_per_step": b2b_us,
        "graph_replay_us_per_step": None if graph_us is None else round(graph_us, 2),
        "graph_vs_eager_b2b_us_per_step": (None if b2b_settled_us is None
                                           else round(b2b_settled_us, 2)),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": (round(value_us / REF_A6000_US, 4)
                        if args.config == "cfg2" and dname == "f32" else None),
        "vs_baseline_ref": "reference kernels, RTX A6000, 16.92 ms (README.md:367)",
        "dtype": dname,
        "kv_cache": "fp8_e4m3" if fp8kv else dname,
        "data": "synthetic",
        "config": {"workload": desc, "B": B, "Sq": Sq, "Sk": Sk, "hidden": dims.hidden,
                   "heads": dims.n_heads, "q_lora": dims.q_lora, "kv_rank": dims.kv_rank,
                   "nope": dims.nope, "rope": dims.rope, "v": dims.v},
        "roofline": roofline,
        "steps_us": per_step,
        "steps_in_layer_us": in_layer_steps,
        "dominant_in_layer": dominant_in_layer,
        "layer_bound_us": round(layer_bound_us, 1),
        "layer_roofline_frac": round(layer_bound_us / value_us, 4),
        "per_step_sum_us": None if steps_sum is None else round(steps_sum, 2),
        # (null where a step has no time: the fp8-cache pass under another profiler)
        "fused_path_sum_us": (round(sum(step_us[n] for n in FUSED_PATH), 2)
                              if fused_attn and not light and all(n in step_us
                                                                  for n in FUSED_PATH)
                              else None),
        "per_step_vs_fused_max_abs": same,
        "neighbours": nb,
        "torch_same_gpu": torch_same,
        "wall_s_timed": round(t_wall, 3),
    }

    if not args.no_cpu_baseline:
        print("[bench] timing the CPU oracle ...", file=sys.stderr, flush=True)
        cb, err, _ = cpu_baseline(inp, out.cpu(), causal=causal)
        rec["cpu_baseline"] = cb
        rec["parity_max_abs_vs_cpu_oracle"] = err
        rec["gpu_speedup_vs_cpu"] = round(cb["value"] / value_us, 1)
    else:
        rec["cpu_baseline"] = None

    return rec


def suite(args, ext, dev):
    """The reference's scenario matrix (SCENARIOS): per scenario the layer through the
    drop-in calls (weights split once, as a serving process holds them) and the same layer
    through torch on this GPU, both timed like the headline (flush read, then the layer
    between events; the reference's own loop, exhaustive_benchmark_suite.py:410-427, flushes
    with a 256 MB write and takes min(10, iters) warm-up calls, as here).  Each scenario first
    checks the layer against the torch result with the reference's suite gate (:466-471).
    Returns one JSON record."""
    import torch
    import mla_inputs

    dims = mla_inputs.DEEPSEEK_V3
    scale = math.sqrt(dims.qk_head)
    flush = torch.zeros(512 << 18, dtype=torch.float32, device=dev)
    names = args.suite_only.split(",") if args.suite_only else list(SCENARIOS)
    rows = []
    settled = False
    for name in names:
        B, Sq, Sk, iters, ref_base, ref_fused = SCENARIOS[name]
        print(f"[suite] {name}: B={B} Sq={Sq} Sk={Sk}", file=sys.stderr, flush=True)
        g = mla_inputs.make_inputs(B, Sq, Sk, seed=args.seed, device=dev)
        W_uk = g["wkv_b"][:, :dims.nope, :].contiguous()
        W_uv = g["wkv_b"][:, dims.nope:, :].contiguous()

        def ours():
            qa, qr = ext.q_absorbed(g["x"], g["W_q_a"], g["q_norm_w"], g["W_q_b"], W_uk,
                                    g["positions"], dims.nope, dims.rope, 1e-6)
            return ext.mla_attention(qa, qr, g["c_kv"], g["pe_cache"], W_uv, scale)

        def base():
            return torch_layer(g, W_uk, W_uv, dims, scale)

        if not settled:
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < args.settle:
                flush.sum()
                ours()
                torch.cuda.synchronize()
            settled = True
        o = ours()
        try:
            b = base()
        except torch.cuda.OutOfMemoryError:
            b = None
        row = {"scenario": name, "phase": "prefill" if Sq > 4 else "decode",
               "B": B, "Sq": Sq, "Sk": Sk, "iters": iters}
        if b is not None:
            tol = dict(rtol=3e-2, atol=3e-2)
            if Sk > 2048:
                tol = dict(rtol=5e-2, atol=max(3e-2, 3e-5 * Sk))
            row["max_abs_diff_vs_torch"] = (o - b).abs().max().item()
            row["max_abs_torch"] = b.abs().max().item()
            row["gate_pass"] = bool(torch.allclose(b, o, **tol))
            del b
        del o
        torch.cuda.empty_cache()
        ours_ms = time_flushed(ours, iters, min(10, iters), flush)
        try:
            base_ms = time_flushed(base, iters, min(10, iters), flush)
        except torch.cuda.OutOfMemoryError:
            base_ms = None
        torch.cuda.empty_cache()
        w = step_work(B, Sq, Sk, dims)
        fl = sum(w[k][0] for k in ("2a1", "2a-n", "2a2", "2b", "2c", "3abc", "3d"))
        row.update({"layer_ms": round(ours_ms, 4),
                    "layer_tflops": round(fl / (ours_ms * 1e-3) / 1e12, 1),
                    "layer_mfma_pct": round(100 * fl / (ours_ms * 1e-3) / PEAK_F32, 1),
                    "torch_ms": None if base_ms is None else round(base_ms, 4),
                    "torch_over_layer": None if base_ms is None else round(base_ms / ours_ms, 3),
                    "a6000_baseline_ms": ref_base, "a6000_fused_ms": ref_fused,
                    "a6000_fused_over_layer": (None if ref_fused is None
                                               else round(ref_fused / ours_ms, 2))})
        print(f"[suite]   layer {ours_ms:.3f} ms ({row['layer_mfma_pct']}% fp32 MFMA), torch "
              f"{base_ms if base_ms is None else round(base_ms, 3)} ms, A6000 fused {ref_fused} ms",
              file=sys.stderr, flush=True)
        rows.append(row)
        del g, W_uk, W_uv
        torch.cuda.empty_cache()

    def gmean(xs):
        xs = [x for x in xs if x]
        return round(math.exp(sum(math.log(x) for x in xs) / len(xs)), 3) if xs else None

    return {"suite": "reference scenario matrix (exhaustive_benchmark_suite.py:78-174)",
            "unit": "ms per layer", "dtype": "f32", "n_gpus": 1, "data": "synthetic",
            "rows": rows,
            "geomean_torch_over_layer": gmean([r["torch_over_layer"] for r in rows]),
            "geomean_a6000_fused_over_layer": gmean([r["a6000_fused_over_layer"] for r in rows]),
            "all_gates_pass": all(r.get("gate_pass", True) for r in rows)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle", type=float, default=2.0, metavar="SECONDS",
                    help="seconds of untimed flush-then-layer loop before the warm-up "
                         "layers, so the clock has settled (see measure())")
    ap.add_argument("--no-bf16-line", action="store_true",
                    help="cfg2 only: skip the bf16 cfg4 figures added to its JSON line")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="cfg2 only: skip the other BASELINE configurations (cfg1, B=1/8/32, "
                         "cfg5) added to its JSON line")
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS))
    ap.add_argument("--dtype", default=None, choices=["f32", "bf16", "f16"],
                    help="storage/MFMA dtype (default: f32, bf16 for cfg4)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kv-cache", default="same", choices=["same", "fp8"],
                    help="cache format of the timed layer: the storage dtype, or fp8 e4m3 with "
                         "a per-tensor scale (bf16 queries only)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--graph-compare", action="store_true",
                    help="only time eager back-to-back layers against HIP-graph replays of the "
                         "same layer (after a settle), marker kernels between the regions")
    ap.add_argument("--suite", action="store_true",
                    help="run the reference's scenario matrix instead (fp32; the layer and "
                         "torch's formulation on this GPU per scenario); one JSON line")
    ap.add_argument("--suite-only", default="", metavar="NAMES",
                    help="comma-separated scenario names for --suite (default: all)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES, 3 times (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against a known byte count)")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="JSON of HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by a 1 GiB copy calibration")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE={world}).", file=sys.stderr)
        sys.exit(2)

    import torch
    import mla_custom_cuda as ext
    import mla_inputs

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        src = torch.empty(args.copy_probe // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": args.copy_probe}), flush=True)
        return
    if args.suite:
        print(json.dumps(suite(args, ext, dev)), flush=True)
        return
    rec = measure(args, ext, dev)
    if args.graph_compare:
        print(json.dumps(rec), flush=True)
        return
    if args.config == "cfg2" and (args.dtype or "f32") == "f32" and not args.no_bf16_line:
        # the bf16 decode (cfg4) beside the headline fp32 one: its layer time and the fused
        # attention's roofline, measured the same way (neighbours and CPU baseline left out)
        a4 = argparse.Namespace(**vars(args))
        a4.config, a4.dtype, a4.no_cpu_baseline = "cfg4", "bf16", True
        r4 = measure(a4, ext, dev, neighbours=False)
        rec["bf16_cfg4"] = {k: r4[k] for k in ("value", "unit", "median_us_per_step",
                                               "back_to_back_us_per_step", "dtype", "config",
                                               "roofline", "fused_path_sum_us")}
        rec["bf16_cfg4"]["steps_us_3abc"] = r4["steps_us"]["3abc"]
        for k in ("steps_in_layer_us", "dominant_in_layer", "layer_bound_us",
                  "layer_roofline_frac"):
            rec["bf16_cfg4"][k] = r4[k]
        # the same layer with the cache held as fp8 E4M3 codes (one per-tensor scale): the
        # cache-format neighbour of the path, its layer time and fused-pass roofline
        a8 = argparse.Namespace(**vars(a4))
        a8.kv_cache = "fp8"
        a8.settle = min(args.settle, 1.0)
        r8 = measure(a8, ext, dev, neighbours=False, light=True)
        rec["fp8kv_cfg4"] = {k: r8[k] for k in ("value", "unit", "median_us_per_step",
                                                "back_to_back_us_per_step", "dtype", "kv_cache",
                                                "config", "roofline", "steps_in_layer_us",
                                                "dominant_in_layer")}
    if args.config == "cfg2" and (args.dtype or "f32") == "f32" and not args.no_other_configs:
        # every other BASELINE configuration, fp32, timed the same way (flushed layers after
        # a settle), with its in-layer kernel times, its fused attention's roofline and the
        # layer's own roofline fraction: cfg1 (B=1, Sk=512), the small-batch sweep B = 1, 8,
        # 32 at Sk=4989, and the causal chunked prefill cfg5 (B=4, Sq=128, Sk=32768)
        rec["other_configs"] = {}
        for name in ("cfg1", "b1", "b8", "b32", "cfg5"):
            a = argparse.Namespace(**vars(args))
            a.config, a.dtype, a.no_cpu_baseline = name, "f32", True
            a.settle = min(args.settle, 1.0)
            if name == "cfg5":     # ~34 ms layers
                a.steps, a.warmup = min(args.steps, 5), min(args.warmup, 2)
            r = measure(a, ext, dev, neighbours=False, light=True)
            rec["other_configs"][name] = {k: r[k] for k in (
                "value", "unit", "median_us_per_step", "back_to_back_us_per_step", "steps",
                "dtype", "config", "roofline", "steps_in_layer_us", "dominant_in_layer",
                "layer_bound_us", "layer_roofline_frac")}
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
