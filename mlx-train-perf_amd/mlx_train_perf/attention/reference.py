"""Materialized attention, `impl="reference"` (mirror of src/mlx_train_perf/attention/reference.py).

`math_attention` builds the full (N, N) scores in fp32, softmaxes and multiplies into V; autograd
differentiates through it. `flash_attention_reference` returns (O, L) with L the fp32 row
logsumexp. GQA: query head h reads kv head h // (Hq // Hkv). An explicit opt-in for small N only;
never chosen by `impl="auto"`.
"""
from __future__ import annotations

import torch

from mlx_train_perf.attention.segments import PackedMask, segment_allowed


def kv_head_for(q_head: int, group_size: int) -> int:
    """Contiguous GQA grouping (reference.py:37-39)."""
    return q_head // group_size


def _masked_scaled_scores(q, k, v, *, scale, causal, segments=None):
    hq, hkv = q.shape[1], k.shape[1]
    if hq % hkv != 0:
        raise ValueError(f"Hq={hq} must be a multiple of Hkv={hkv} for GQA grouping")
    group = hq // hkv
    idx = torch.tensor([kv_head_for(h, group) for h in range(hq)], device=q.device)
    q32 = q.to(torch.float32)
    k_g = k.index_select(1, idx).to(torch.float32)
    v_g = v.index_select(1, idx).to(torch.float32)
    scores = (q32 @ k_g.transpose(-1, -2).contiguous()) * scale
    n = q.shape[2]
    if segments is not None:
        assert causal, "segments requires causal=True"
        return scores.masked_fill(~segment_allowed(segments.seg_id), float("-inf")), v_g
    if causal:
        tri = torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1)
        scores = scores.masked_fill(tri, float("-inf"))
    return scores, v_g


def _attention_core(q, k, v, *, scale, causal, segments=None):
    scores, v_g = _masked_scaled_scores(q, k, v, scale=scale, causal=causal, segments=segments)
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.exp(scores - lse[..., None])
    o = (probs @ v_g).to(q.dtype)
    return o, lse


def math_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, causal: bool = True,
                   segments: PackedMask | None = None) -> torch.Tensor:
    o, _ = _attention_core(q, k, v, scale=scale, causal=causal, segments=segments)
    return o


def flash_attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float,
                              causal: bool = True, segments: PackedMask | None = None):
    return _attention_core(q, k, v, scale=scale, causal=causal, segments=segments)
