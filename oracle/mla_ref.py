"""CPU restatement of the reference's absorbed MLA layer -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only as the checker or the timed CPU baseline.  The product
path (``libmla_amd.so`` and the ``mla_custom_cuda`` extension) never calls into it.

What it restates (reference = pgangwar-ucsd/mla-cuda):

* the end-to-end PyTorch formulation the reference checks its kernels against,
  ``exhaustive_benchmark_suite.py:210-304`` (``apply_rope``, ``rmsnorm``,
  ``split_wkv_b``, ``prepare_q_mla_absorbed``, ``mla_attention_official``) and its
  composition ``baseline_official_mla_attention`` (``:387-390``);
* the per-step decomposition the reference's kernels compute
  (``mla_kernels.cu`` steps 2a1, 2a-n, 2a2, 2b, 2c, 3a, 3b, 3c, 3d), so every
  intermediate the HIP path produces has an oracle value: the split softmax of 3a/3b
  (``mla_kernels.cu:971-1032, 1058-1079``), the unnormalised ctx of 3c
  (``:1101-1118``) and the deferred divide in 3d (``:1385-1415``);
* one extension the reference does not have: a causal mask (key j visible to query i iff
  j <= Sk - Sq + i), used by the chunked-prefill configuration;
* the path's neighbours, which the reference names but does not implement: the KV-cache
  append (``kv_append``) and the output projection (``o_proj``);
* a ragged, paged cache (``gather_pages``, ``mla_attention_paged``, ``prepare_q_ragged``,
  ``kv_append_paged``): the same per-sequence math over keys found through a page table;
* an fp8 cache (``e4m3_values``, ``decode_e4m3``, ``mla_attention_fp8kv``): OCP float8
  E4M3 codes of value / kv_scale, decoded and then the same attention in float32.

Arithmetic runs in torch on the CPU, in float32 for float32/bfloat16/float16 inputs and in
float64 for float64 inputs -- the reference's accumulate-dtype policy
(``mla_kernels.cu:115-120``).

Every function here is pinned by ``tests/test_oracle.py`` against an independent
brute-force loop implementation on tiny shapes, closed forms (RoPE rotation, RMS of the
norm output) and invariants (softmax normalisation, split-softmax == direct softmax,
causal Sq=1 == non-causal).  No reference golden vectors exist (the reference commits
none); those checks are what pins each function.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

# ---------------------------------------------------------------------------
# Model dimensions -- exhaustive_benchmark_suite.py:30-49 (DeepSeekV3Config)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class MLADims:
    hidden: int = 7168
    n_heads: int = 128
    q_lora: int = 1536
    kv_rank: int = 512
    nope: int = 128
    rope: int = 64
    v: int = 128

    @property
    def qk_head(self) -> int:  # exhaustive_benchmark_suite.py:41-42
        return self.nope + self.rope

    @property
    def q_absorbed(self) -> int:  # exhaustive_benchmark_suite.py:45-47
        return self.kv_rank + self.rope


DSV3 = MLADims()
RMS_NORM_EPS = 1e-6          # exhaustive_benchmark_suite.py:249
ROPE_BASE = 10000.0          # exhaustive_benchmark_suite.py:218
SCORE_TILE = 128             # keys per softmax partial (mla_kernels.cu:63, 1543)


def acc_dtype(dtype: torch.dtype) -> torch.dtype:
    """Accumulate dtype: float64 stays float64, everything else is float32
    (mla_kernels.cu:115-120; exhaustive_benchmark_suite.py:214, 254)."""
    return torch.float64 if dtype == torch.float64 else torch.float32


# ---------------------------------------------------------------------------
# End-to-end formulation (the reference's PyTorch oracle)
# ---------------------------------------------------------------------------


def rope_inv_freq(rope_dim: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """1 / base^(2i/rope_dim) for i < rope_dim/2, evaluated in ``dtype`` exactly the way
    exhaustive_benchmark_suite.py:216-219 evaluates it (torch CPU pow in that dtype).
    The HIP path receives this very table, so kernel and oracle angles are bit-equal."""
    expo = torch.arange(0, rope_dim, 2, dtype=dtype) / rope_dim
    return 1.0 / (ROPE_BASE ** expo)


def apply_rope(x: torch.Tensor, positions: torch.Tensor, rope_dim: int) -> torch.Tensor:
    """Interleaved-pair rotary embedding over the last dim of x [B, Sq, H, rope_dim].

    Pair (2i, 2i+1) at position p is rotated by p * inv_freq[i]
    (exhaustive_benchmark_suite.py:210-232): even' = e*cos - o*sin, odd' = e*sin + o*cos.
    cos/sin are rounded to x's dtype before use, the rotation runs in the acc dtype and
    the result is rounded back to x's dtype.
    """
    acc = acc_dtype(x.dtype)
    inv_freq = rope_inv_freq(rope_dim, acc)
    ang = torch.outer(positions.to(acc), inv_freq)                     # [Sq, rope/2]
    half = rope_dim // 2
    c = torch.cos(ang).to(x.dtype).to(acc).reshape(1, -1, 1, half)
    s = torch.sin(ang).to(x.dtype).to(acc).reshape(1, -1, 1, half)
    xa = x.to(acc)
    ev, od = xa[..., 0::2], xa[..., 1::2]
    rot = torch.empty_like(xa)
    rot[..., 0::2] = ev * c - od * s
    rot[..., 1::2] = ev * s + od * c
    return rot.to(x.dtype)


def rmsnorm(x: torch.Tensor, gain: torch.Tensor, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps), rounded to x's dtype, times the gain
    (exhaustive_benchmark_suite.py:252-258)."""
    acc = acc_dtype(x.dtype)
    xa = x.to(acc)
    inv = torch.rsqrt(xa.square().mean(dim=-1, keepdim=True) + eps)
    return (xa * inv).to(x.dtype) * gain


def split_wkv_b(wkv_b: torch.Tensor, nope: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """wkv_b [H, nope+v, R] -> (W_uk [H, nope, R], W_uv [H, v, R]) views
    (exhaustive_benchmark_suite.py:261-265)."""
    return wkv_b[:, :nope, :], wkv_b[:, nope:, :]


def prepare_q_mla_absorbed(x, W_q_a, q_norm_w, W_q_b, W_uk, positions,
                           nope: int, rope: int, eps: float = RMS_NORM_EPS):
    """x [B,Sq,hidden] -> (q_absorbed [B,Sq,H,R], q_rope [B,Sq,H,rope])
    (exhaustive_benchmark_suite.py:268-286)."""
    B, Sq, _ = x.shape
    H = W_uk.shape[0]
    lat = rmsnorm(torch.matmul(x, W_q_a), q_norm_w, eps)
    q = torch.matmul(lat, W_q_b).reshape(B, Sq, H, nope + rope)
    q_nope, q_pe = q[..., :nope], q[..., nope:]
    # per-head absorption  q_abs[b,s,h,:] = q_nope[b,s,h,:] @ W_uk[h]
    q_abs = torch.matmul(q_nope.permute(2, 0, 1, 3).reshape(H, B * Sq, nope), W_uk)
    q_abs = q_abs.reshape(H, B, Sq, -1).permute(1, 2, 0, 3).contiguous()
    return q_abs, apply_rope(q_pe, positions, rope)


def causal_mask(Sq: int, Sk: int) -> torch.Tensor:
    """[Sq, Sk] bool, True where key j is visible to query i: j <= Sk - Sq + i.
    (Not in the reference; the chunked-prefill configuration asks for it.)"""
    qi = torch.arange(Sq).unsqueeze(1)
    kj = torch.arange(Sk).unsqueeze(0)
    return kj <= (Sk - Sq + qi)


def mla_attention_official(q_absorbed, q_rope, c_kv, pe_cache, W_uv, scale: float,
                           causal: bool = False):
    """softmax((q_abs . c_kv + q_rope . pe) / scale) @ c_kv, then @ W_uv^T
    (exhaustive_benchmark_suite.py:289-304).  ``scale`` is a divisor (the reference
    passes sqrt(192), :298, :328).  Shapes: q_absorbed [B,Sq,H,R], q_rope [B,Sq,H,D],
    c_kv [B,Sk,R], pe_cache [B,Sk,D], W_uv [H,V,R] -> [B,Sq,H,V]."""
    B, Sq, H, R = q_absorbed.shape
    Sk = c_kv.shape[1]
    qa = q_absorbed.reshape(B, Sq * H, R)
    qr = q_rope.reshape(B, Sq * H, -1)
    s = (torch.bmm(qa, c_kv.transpose(1, 2).contiguous())
         + torch.bmm(qr, pe_cache.transpose(1, 2).contiguous())) / scale   # [B,Sq*H,Sk]
    if causal:
        vis = causal_mask(Sq, Sk).repeat_interleave(H, dim=0)              # [Sq*H, Sk]
        s = s.masked_fill(~vis.unsqueeze(0), float("-inf"))
    attn = torch.softmax(s, dim=-1)
    ctx = torch.bmm(attn, c_kv).reshape(B, Sq, H, R)                       # [B,Sq,H,R]
    out = torch.matmul(ctx.permute(2, 0, 1, 3).reshape(H, B * Sq, R),
                       W_uv.transpose(1, 2).contiguous())                  # [H,B*Sq,V]
    return out.reshape(H, B, Sq, -1).permute(1, 2, 0, 3).contiguous()


def mla_layer(x, W_q_a, q_norm_w, W_q_b, wkv_b, c_kv, pe_cache, positions,
              dims: MLADims = DSV3, eps: float = RMS_NORM_EPS, causal: bool = False,
              scale: Optional[float] = None):
    """Whole layer 2a1 -> 3d (exhaustive_benchmark_suite.py:387-390)."""
    W_uk, W_uv = split_wkv_b(wkv_b, dims.nope)
    qa, qr = prepare_q_mla_absorbed(x, W_q_a, q_norm_w, W_q_b, W_uk, positions,
                                    dims.nope, dims.rope, eps)
    if scale is None:
        scale = float(dims.qk_head) ** 0.5
    return mla_attention_official(qa, qr, c_kv, pe_cache, W_uv, scale, causal)


# ---------------------------------------------------------------------------
# Per-step decomposition (what each HIP kernel must produce)
# ---------------------------------------------------------------------------


def step_gemm(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """2a1 / 2a2: a [M,K] @ w [K,N] in the acc dtype (mla_kernels.cu:233-366)."""
    acc = acc_dtype(a.dtype)
    return torch.matmul(a.to(acc), w.to(acc))


def step_norm(q_lat_acc: torch.Tensor, gain: torch.Tensor, eps: float,
              out_dtype: torch.dtype) -> torch.Tensor:
    """2a-n: RMSNorm of the acc-dtype latent, gain applied in the acc dtype, then
    narrowed to the input dtype (mla_kernels.cu:377-420)."""
    acc = q_lat_acc.dtype
    inv = torch.rsqrt(q_lat_acc.square().mean(dim=-1, keepdim=True) + eps)
    return (q_lat_acc * inv * gain.to(acc)).to(out_dtype)


def step_rope(q_raw: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor,
              B: int, Sq: int, H: int, nope: int, rope: int,
              out_dtype: torch.dtype) -> torch.Tensor:
    """2b: RoPE of q_raw[bq, h*(nope+rope) + nope : +rope] -> [B,Sq,H,rope]
    (mla_kernels.cu:425-466).  Rows bq = b*Sq + s use positions[s] (:449)."""
    acc = q_raw.dtype
    qr = q_raw.reshape(B, Sq, H, nope + rope)[..., nope:]
    ang = torch.outer(positions.to(acc), inv_freq.to(acc))
    half = rope // 2
    c = torch.cos(ang).reshape(1, Sq, 1, half)
    s = torch.sin(ang).reshape(1, Sq, 1, half)
    ev, od = qr[..., 0::2], qr[..., 1::2]
    out = torch.empty(B, Sq, H, rope, dtype=acc)
    out[..., 0::2] = ev * c - od * s
    out[..., 1::2] = ev * s + od * c
    return out.to(out_dtype)


def step_absorb(q_raw: torch.Tensor, W_uk: torch.Tensor, B: int, Sq: int, nope: int,
                out_dtype: torch.dtype) -> torch.Tensor:
    """2c: q_absorbed[b,s,h,:] = q_raw[b,s,h,0:nope] @ W_uk[h] (mla_kernels.cu:474-596)."""
    H, _, R = W_uk.shape
    acc = q_raw.dtype
    qn = q_raw.reshape(B * Sq, H, -1)[..., :nope].permute(1, 0, 2)        # [H,bq,nope]
    qa = torch.bmm(qn.contiguous(), W_uk.to(acc))                         # [H,bq,R]
    return qa.permute(1, 0, 2).reshape(B, Sq, H, R).to(out_dtype)


def step_scores(q_absorbed, q_rope, c_kv, pe_cache, scale: float, tile: int = SCORE_TILE,
                causal: bool = False):
    """3a: s = (q_abs . c_kv + q_rope . pe) * (1/scale) as one 576-deep product; per row
    and per ``tile``-key block j: m_j = max over the block's visible keys, stored
    p = exp(s - m_j) (0 where masked), l_j = sum of p (mla_kernels.cu:808-1033).

    Returns p [flat, Sk], m [flat, P], l [flat, P] with flat = B*Sq*H, P = ceil(Sk/tile).
    A block with no visible key has m = -inf, l = 0."""
    B, Sq, H, R = q_absorbed.shape
    Sk = c_kv.shape[1]
    acc = acc_dtype(q_absorbed.dtype)
    qa = q_absorbed.to(acc).reshape(B, Sq * H, R)
    qr = q_rope.to(acc).reshape(B, Sq * H, -1)
    ck = c_kv.to(acc)
    pe = pe_cache.to(acc)
    inv_scale = torch.tensor(1.0, dtype=acc) / torch.tensor(scale, dtype=acc)
    s = (torch.bmm(qa, ck.transpose(1, 2).contiguous())
         + torch.bmm(qr, pe.transpose(1, 2).contiguous())) * inv_scale
    s = s.reshape(B * Sq * H, Sk)
    if causal:
        vis = causal_mask(Sq, Sk).repeat_interleave(H, dim=0).repeat(B, 1)
    else:
        vis = torch.ones_like(s, dtype=torch.bool)
    P = (Sk + tile - 1) // tile
    pad = P * tile - Sk
    sp = torch.nn.functional.pad(s, (0, pad)).reshape(-1, P, tile)
    vp = torch.nn.functional.pad(vis, (0, pad), value=False).reshape(-1, P, tile)
    m = sp.masked_fill(~vp, float("-inf")).amax(dim=-1)                   # [flat,P]
    msafe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    p = torch.exp(sp - msafe.unsqueeze(-1)).masked_fill(~vp, 0.0)
    l = p.sum(dim=-1)
    return p.reshape(-1, P * tile)[:, :Sk].contiguous(), m, l


def step_combine(m: torch.Tensor, l: torch.Tensor):
    """3b: M = max_j m_j; alpha_j = 1 if m_j == M else exp(m_j - M);
    row_sum = sum_j l_j * alpha_j (mla_kernels.cu:1036-1081)."""
    M = m.amax(dim=-1, keepdim=True)
    alpha = torch.where(m == M, torch.ones_like(m), torch.exp(m - M))
    return alpha, (l * alpha).sum(dim=-1)


def step_ctx(p: torch.Tensor, alpha: torch.Tensor, c_kv: torch.Tensor, B: int, Sq: int,
             H: int, tile: int = SCORE_TILE) -> torch.Tensor:
    """3c: unnormalised ctx[row,:] = sum_k p[row,k] * alpha[row, k//tile] * c_kv[b,k,:]
    (mla_kernels.cu:1101-1326).  Returns [B,Sq,H,R] in the acc dtype."""
    Sk = c_kv.shape[1]
    acc = p.dtype
    a = alpha.repeat_interleave(tile, dim=1)[:, :Sk]
    w = (p * a).reshape(B, Sq * H, Sk)
    return torch.bmm(w, c_kv.to(acc)).reshape(B, Sq, H, -1)


def step_out(ctx: torch.Tensor, row_sum: torch.Tensor, W_uv: torch.Tensor,
             out_dtype: torch.dtype) -> torch.Tensor:
    """3d: out[b,s,h,:] = (ctx[b,s,h,:] * (1/row_sum[b,s,h])) @ W_uv[h]^T
    (mla_kernels.cu:1339-1476)."""
    B, Sq, H, R = ctx.shape
    acc = ctx.dtype
    inv = (1.0 / row_sum).reshape(B, Sq, H, 1)
    cn = (ctx * inv).permute(2, 0, 1, 3).reshape(H, B * Sq, R)
    o = torch.bmm(cn, W_uv.to(acc).transpose(1, 2).contiguous())
    return o.reshape(H, B, Sq, -1).permute(1, 2, 0, 3).to(out_dtype).contiguous()


def layer_by_steps(inp: Dict[str, torch.Tensor], dims: MLADims = DSV3,
                   eps: float = RMS_NORM_EPS, causal: bool = False,
                   tile: int = SCORE_TILE) -> Dict[str, torch.Tensor]:
    """Run all nine steps and return every intermediate (keys named after the steps)."""
    x = inp["x"]
    B, Sq, hidden = x.shape
    dt = x.dtype
    H, nope, rope = dims.n_heads, dims.nope, dims.rope
    W_uk, W_uv = split_wkv_b(inp["wkv_b"], nope)
    acc = acc_dtype(dt)
    r = {}
    r["q_lat_acc"] = step_gemm(x.reshape(B * Sq, hidden), inp["W_q_a"])
    r["q_lat"] = step_norm(r["q_lat_acc"], inp["q_norm_w"], eps, dt)
    r["q_raw"] = step_gemm(r["q_lat"], inp["W_q_b"])
    inv_freq = rope_inv_freq(rope, acc)
    r["q_rope"] = step_rope(r["q_raw"], inp["positions"], inv_freq, B, Sq, H, nope, rope, dt)
    r["q_absorbed"] = step_absorb(r["q_raw"], W_uk, B, Sq, nope, dt)
    scale = float(dims.qk_head) ** 0.5
    r["p"], r["m"], r["l"] = step_scores(r["q_absorbed"], r["q_rope"], inp["c_kv"],
                                         inp["pe_cache"], scale, tile, causal)
    r["alpha"], r["row_sum"] = step_combine(r["m"], r["l"])
    r["ctx"] = step_ctx(r["p"], r["alpha"], inp["c_kv"], B, Sq, H, tile)
    r["out"] = step_out(r["ctx"], r["row_sum"], W_uv, dt)
    return r


# ---------------------------------------------------------------------------
# Neighbours of the path (not in the reference's kernels)
# ---------------------------------------------------------------------------


def kv_append(x: torch.Tensor, W_kv_a: torch.Tensor, kv_norm_w: torch.Tensor,
              positions: torch.Tensor, c_kv: torch.Tensor, pe_cache: torch.Tensor,
              start_row: int, eps: float = RMS_NORM_EPS) -> Tuple[torch.Tensor, torch.Tensor]:
    """KV-cache write of the absorbed layout.  The reference describes it without
    implementing it (exhaustive_benchmark_suite.py:188-196): ``wkv_a`` maps x to
    [c_kv, k_pe_raw] for the cache write, and pe_cache holds K_rope after RoPE.  The
    algorithm is DeepSeek-V3's published one (deepseek-ai/DeepSeek-V3, inference/model.py,
    MLA.forward, absorb branch; a third-party source the reference does not vendor, no
    pinned version): kv = x @ wkv_a; kv_cache[:, start:end] = kv_norm(kv[..., :kv_rank]);
    pe_cache[:, start:end] = rotary(kv[..., kv_rank:]) at the token positions.

    Arithmetic follows this path's Q-side steps: the product in the acc dtype
    (``step_gemm``), the norm of the acc-dtype latent with the gain applied before
    narrowing (``step_norm``), and the interleaved-pair rotation of the acc-dtype rope
    columns (``step_rope`` with one head).  Returns updated copies of the two caches."""
    B, Sq, hidden = x.shape
    R, D = c_kv.shape[-1], pe_cache.shape[-1]
    dt = x.dtype
    kv = step_gemm(x.reshape(B * Sq, hidden), W_kv_a)                    # [B*Sq, R + D]
    lat = step_norm(kv[:, :R], kv_norm_w, eps, dt).reshape(B, Sq, R)
    inv_freq = rope_inv_freq(D, acc_dtype(dt))
    kpe = step_rope(kv, positions, inv_freq, B, Sq, 1, R, D, dt).reshape(B, Sq, D)
    c2, p2 = c_kv.clone(), pe_cache.clone()
    c2[:, start_row:start_row + Sq] = lat
    p2[:, start_row:start_row + Sq] = kpe
    return c2, p2


def o_proj(attn: torch.Tensor, W_o: torch.Tensor) -> torch.Tensor:
    """Output projection wo, the step after the layer's output [B, Sq, H, v] (named by the
    reference's scope, not implemented there): [B*Sq, H*v] @ W_o [H*v, hidden] in the acc
    dtype, narrowed to the input dtype."""
    B, Sq, H, v = attn.shape
    return step_gemm(attn.reshape(B * Sq, H * v), W_o).to(attn.dtype).reshape(B, Sq, -1)


# ---------------------------------------------------------------------------
# Ragged, paged KV cache (the reference's cache is one dense [B, Sk] block with one Sk
# and query positions shared by the batch: mla_kernels.cu:1489, 847-848, 449)
# ---------------------------------------------------------------------------


def gather_pages(pages: torch.Tensor, table_row: torch.Tensor, n: int) -> torch.Tensor:
    """Keys [0, n) of one sequence from a paged pool [num_pages, page_size, width]: key k
    is row k % page_size of page table_row[k // page_size]."""
    page = pages.shape[1]
    k = torch.arange(n)
    return pages[table_row.long()[k // page], k % page]


def mla_attention_paged(q_absorbed, q_rope, c_kv_pages, pe_pages, block_table, seq_lens,
                        W_uv, scale: float, causal: bool = False) -> torch.Tensor:
    """Each sequence b attends, exactly as ``mla_attention_official`` (the reference's
    formulation, exhaustive_benchmark_suite.py:282-304), to its own seq_lens[b] keys
    gathered from the pages; the causal rule is relative to that length."""
    outs = []
    for b in range(q_absorbed.shape[0]):
        n = int(seq_lens[b])
        ck = gather_pages(c_kv_pages, block_table[b], n).unsqueeze(0)
        pe = gather_pages(pe_pages, block_table[b], n).unsqueeze(0)
        outs.append(mla_attention_official(q_absorbed[b:b + 1], q_rope[b:b + 1], ck, pe, W_uv,
                                           scale, causal))
    return torch.cat(outs)


def prepare_q_ragged(x, W_q_a, q_norm_w, W_q_b, W_uk, positions, nope: int, rope: int,
                     eps: float = RMS_NORM_EPS):
    """``prepare_q_mla_absorbed`` with per-sequence positions [B, Sq]: sequence b's query
    rows use row b of positions."""
    qa, qr = [], []
    for b in range(x.shape[0]):
        a, r = prepare_q_mla_absorbed(x[b:b + 1], W_q_a, q_norm_w, W_q_b, W_uk, positions[b],
                                      nope, rope, eps)
        qa.append(a); qr.append(r)
    return torch.cat(qa), torch.cat(qr)


def kv_append_paged(x, W_kv_a, kv_norm_w, positions, block_table, c_kv_pages, pe_pages,
                    eps: float = RMS_NORM_EPS) -> Tuple[torch.Tensor, torch.Tensor]:
    """``kv_append`` into a paged cache: token (b, s) goes to slot positions[b, s] of
    sequence b, i.e. row slot % page_size of page block_table[b, slot // page_size];
    slots outside the table are skipped.  Returns updated copies of the two pools."""
    B, Sq, _ = x.shape
    R, D = c_kv_pages.shape[-1], pe_pages.shape[-1]
    page, max_pages = c_kv_pages.shape[1], block_table.shape[1]
    c2, p2 = c_kv_pages.clone(), pe_pages.clone()
    for b in range(B):
        dc = torch.zeros(1, Sq, R, dtype=c_kv_pages.dtype)
        dp = torch.zeros(1, Sq, D, dtype=pe_pages.dtype)
        rc, rp = kv_append(x[b:b + 1], W_kv_a, kv_norm_w, positions[b], dc, dp, 0, eps)
        for s in range(Sq):
            slot = int(positions[b, s])
            if slot < 0 or slot // page >= max_pages:
                continue
            pg = int(block_table[b, slot // page])
            c2[pg, slot % page] = rc[0, s]
            p2[pg, slot % page] = rp[0, s]
    return c2, p2


# ---------------------------------------------------------------------------
# Seeded synthetic inputs
# ---------------------------------------------------------------------------


def make_inputs(B: int, Sq: int, Sk: int, dims: MLADims = DSV3, seed: int = 0,
                dtype: torch.dtype = torch.float32) -> Dict[str, torch.Tensor]:
    """Seeded CPU inputs in a fixed generation order:
    hidden ~N(0,1); W_q_a ~N(0,1/hidden); q_norm_w = 1 + 0.1 N(0,1) (the reference's gain
    jitter, exhaustive_benchmark_suite.py:363-365); W_q_b ~N(0,1/q_lora);
    wkv_b ~N(0,1/kv_rank); c_kv ~N(0,1); pe_cache ~N(0,1);
    positions = arange(Sk-Sq, Sk) (:383).  Generated in float32 and rounded to ``dtype``
    (float64 inputs are generated in float64)."""
    g = torch.Generator().manual_seed(seed)
    gdt = torch.float64 if dtype == torch.float64 else torch.float32

    def rn(*shape, std=1.0):
        t = torch.randn(*shape, generator=g, dtype=gdt)
        if std != 1.0:
            t.mul_(std)
        return t.to(dtype)

    d = dims
    inp = {}
    inp["x"] = rn(B, Sq, d.hidden)
    inp["W_q_a"] = rn(d.hidden, d.q_lora, std=1.0 / math.sqrt(d.hidden))
    inp["q_norm_w"] = (1.0 + 0.1 * torch.randn(d.q_lora, generator=g, dtype=gdt)).to(dtype)
    inp["W_q_b"] = rn(d.q_lora, d.n_heads * d.qk_head, std=1.0 / math.sqrt(d.q_lora))
    inp["wkv_b"] = rn(d.n_heads, d.nope + d.v, d.kv_rank, std=1.0 / math.sqrt(d.kv_rank))
    inp["c_kv"] = rn(B, Sk, d.kv_rank)
    inp["pe_cache"] = rn(B, Sk, d.rope)
    inp["positions"] = torch.arange(Sk - Sq, Sk, dtype=torch.int64)
    return inp


# ---------------------------------------------------------------------------
# fp8 (OCP E4M3) cache
# ---------------------------------------------------------------------------


def e4m3_values() -> torch.Tensor:
    """The 256 values of the OCP 8-bit floating point format E4M3 (OCP "8-bit Floating Point
    Specification (OFP8)" v1.0), indexed by code: sign bit 7, a 4-bit exponent with bias 7 in
    bits 6-3, a 3-bit mantissa in bits 2-0.  Exponent field 0 holds the subnormals
    m/8 * 2^-6; codes 0x7F and 0xFF are NaN; there are no infinities (the largest finite
    magnitude is 448).  torch.float8_e4m3fn is this format."""
    out = torch.empty(256, dtype=torch.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            out[code] = float("nan")
        elif e == 0:
            out[code] = sign * (m / 8.0) * 2.0 ** -6
        else:
            out[code] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out.float()


_E4M3 = None


def decode_e4m3(codes: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """float32 values code * scale of a uint8 (or float8_e4m3fn) tensor of E4M3 codes."""
    global _E4M3
    if _E4M3 is None:
        _E4M3 = e4m3_values()
    if codes.dtype != torch.uint8:
        codes = codes.view(torch.uint8)
    return _E4M3[codes.long()] * scale


def mla_attention_fp8kv(q_absorbed, q_rope, c_kv_codes, pe_codes, kv_scale: float, W_uv,
                        scale: float, causal: bool = False):
    """mla_attention_official on the decoded fp8 cache (code * kv_scale), in float32 on the
    queries' and W_uv's values."""
    return mla_attention_official(q_absorbed.float(), q_rope.float(),
                                  decode_e4m3(c_kv_codes, kv_scale),
                                  decode_e4m3(pe_codes, kv_scale), W_uv.float(), scale, causal)
