"""Seeded synthetic inputs for the absorbed-MLA layer (used by bench.py).

Generation order and distributions (seeded CPU generator, float32, then rounded to the
requested storage dtype):
  x [B,Sq,hidden] ~N(0,1); W_q_a [hidden,q_lora] ~N(0,1/hidden);
  q_norm_w [q_lora] = 1 + 0.1 N(0,1) (the reference's gain jitter,
  exhaustive_benchmark_suite.py:363-365); W_q_b [q_lora, H*(nope+rope)] ~N(0,1/q_lora);
  wkv_b [H, nope+v, kv_rank] ~N(0,1/kv_rank); c_kv [B,Sk,kv_rank] ~N(0,1);
  pe_cache [B,Sk,rope] ~N(0,1); positions = arange(Sk-Sq, Sk) (:383).
The test suite checks that these tensors are bit-identical to the CPU oracle's inputs.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional

import torch


@dataclass(frozen=True)
class Dims:
    hidden: int = 7168
    n_heads: int = 128
    q_lora: int = 1536
    kv_rank: int = 512
    nope: int = 128
    rope: int = 64
    v: int = 128

    @property
    def qk_head(self) -> int:
        return self.nope + self.rope


DEEPSEEK_V3 = Dims()


def make_inputs(B: int, Sq: int, Sk: int, dims: Dims = DEEPSEEK_V3, seed: int = 0,
                dtype: torch.dtype = torch.float32,
                device: Optional[torch.device] = None) -> Dict[str, torch.Tensor]:
    """With ``device`` the tensors are drawn there by that device's generator (same
    distributions and order, different values): fast set-up of large shapes for timing."""
    g = torch.Generator(device=device) if device is not None else torch.Generator()
    g.manual_seed(seed)

    def normal(*shape, std=1.0):
        t = torch.randn(*shape, generator=g, dtype=torch.float32, device=device)
        if std != 1.0:
            t.mul_(std)
        return t.to(dtype)

    d = dims
    out = {
        "x": normal(B, Sq, d.hidden),
        "W_q_a": normal(d.hidden, d.q_lora, std=1.0 / math.sqrt(d.hidden)),
    }
    out["q_norm_w"] = (1.0 + 0.1 * torch.randn(d.q_lora, generator=g, device=device)).to(dtype)
    out["W_q_b"] = normal(d.q_lora, d.n_heads * d.qk_head, std=1.0 / math.sqrt(d.q_lora))
    out["wkv_b"] = normal(d.n_heads, d.nope + d.v, d.kv_rank, std=1.0 / math.sqrt(d.kv_rank))
    out["c_kv"] = normal(B, Sk, d.kv_rank)
    out["pe_cache"] = normal(B, Sk, d.rope)
    out["positions"] = torch.arange(Sk - Sq, Sk, dtype=torch.int64, device=device)
    return out
