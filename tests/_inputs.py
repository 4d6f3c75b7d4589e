"""Seeded synthetic inputs shared by the tests (the reference's published workload shapes, scaled
down where noted)."""
from __future__ import annotations

import torch


def lce_inputs(n: int, d: int, v: int, *, seed: int = 0, ignore_frac: float = 0.1, w_std: float = 0.02,
               rms_norm: bool = False, ignore_index: int = -100):
    """H ~ N(0,1) (optionally RMS-normalized per row), W ~ N(0, w_std^2), both bf16; targets uniform in
    [0, V) with round(ignore_frac * n) rows (picked by a seeded permutation) set to ignore_index."""
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g)
    if rms_norm:
        h = h / torch.sqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)
    w = torch.randn(v, d, generator=g) * w_std
    t = torch.randint(0, v, (n,), generator=g)
    k = int(round(ignore_frac * n))
    if k:
        t[torch.randperm(n, generator=g)[:k]] = ignore_index
    return h.to(torch.bfloat16), w.to(torch.bfloat16), t


def attn_inputs(b: int, hq: int, hkv: int, s: int, d: int, *, seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, s, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, hkv, s, d, generator=g).to(torch.bfloat16)
    v = torch.randn(b, hkv, s, d, generator=g).to(torch.bfloat16)
    do = torch.randn(b, hq, s, d, generator=g).to(torch.bfloat16)
    return q, k, v, do


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double()
    b = b.double()
    return float((a - b).norm() / b.norm().clamp(min=1e-30))
