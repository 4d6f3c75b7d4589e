"""CPU restatement of the reference's attention oracles (test infrastructure only).

Follows src/mlx_train_perf/attention/reference.py:37-116 (forward) and
src/mlx_train_perf/attention/api.py:126-194 (backward), src/mlx_train_perf/attention/segments.py:22-29
(packed mask):
- layouts q (B, Hq, N, D), k/v (B, Hkv, N, D), O like q, L (B, Hq, N) fp32;
- GQA: query head h reads kv head h // (Hq // Hkv) (reference.py:37-39);
- scores = scale * q @ k^T in fp32 (upcast inputs), causal -inf above the diagonal, packed mode
  replaces the triangle with `segment_allowed` (same segment and j <= i);
- L = logsumexp over keys, P = exp(S - L), O = P @ V;
- backward: D = rowsum(dO * O), dV = P^T dO, dP = dO V^T, dS = P (dP - D), dQ = scale dS K,
  dK = scale dS^T Q, dK and dV summed over each kv head's query-head group.
"""
from __future__ import annotations

import torch


def kv_head_for(q_head: int, group_size: int) -> int:
    """Contiguous GQA grouping (attention/reference.py:37-39)."""
    return q_head // group_size


def segment_allowed(seg_id: torch.Tensor) -> torch.Tensor:
    """(B, 1, N, N) bool: key j visible to query i iff same segment and j <= i (segments.py:22-29)."""
    same = seg_id[:, None, :, None] == seg_id[:, None, None, :]
    n = seg_id.shape[-1]
    causal = torch.tril(torch.ones(n, n, dtype=torch.bool, device=seg_id.device))[None, None]
    return same & causal


def _gather_kv(x: torch.Tensor, hq: int) -> torch.Tensor:
    hkv = x.shape[1]
    idx = torch.tensor([kv_head_for(h, hq // hkv) for h in range(hq)], device=x.device)
    return x.index_select(1, idx)


def _scores(q, k, *, scale, causal, seg_id, dtype):
    hq = q.shape[1]
    if hq % k.shape[1]:
        raise ValueError("Hq must be a multiple of Hkv")
    s = (q.to(dtype) @ _gather_kv(k, hq).to(dtype).transpose(-1, -2).contiguous()) * scale
    n = q.shape[2]
    if seg_id is not None:
        if not causal:
            raise ValueError("segments require causal=True")
        s = s.masked_fill(~segment_allowed(seg_id), float("-inf"))
    elif causal:
        s = s.masked_fill(~torch.tril(torch.ones(n, n, dtype=torch.bool, device=q.device)), float("-inf"))
    return s


def attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, causal: bool = True,
                      seg_id: torch.Tensor | None = None,
                      dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, L) in `dtype` (attention/reference.py:77-116): O = softmax(masked scaled scores) @ V."""
    s = _scores(q, k, scale=scale, causal=causal, seg_id=seg_id, dtype=dtype)
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    o = p @ _gather_kv(v, q.shape[1]).to(dtype)
    return o, lse


def attention_backward(q, k, v, o, lse, d_o, *, scale: float, causal: bool = True,
                       seg_id: torch.Tensor | None = None, dtype: torch.dtype = torch.float32):
    """(dQ, dK, dV) in `dtype` by the FlashAttention equations over full tensors (api.py:140-194)."""
    b, hq, n, dd = q.shape
    hkv = k.shape[1]
    grp = hq // hkv
    q32, o32, do32 = q.to(dtype), o.to(dtype), d_o.to(dtype)
    kg = _gather_kv(k, hq).to(dtype)
    vg = _gather_kv(v, hq).to(dtype)
    dvec = (do32 * o32).sum(-1)
    s = _scores(q, k, scale=scale, causal=causal, seg_id=seg_id, dtype=dtype)
    p = torch.exp(s - lse.to(dtype)[..., None])
    dp = do32 @ vg.transpose(-1, -2).contiguous()
    ds = p * (dp - dvec[..., None])
    dq = scale * (ds @ kg)
    dv_h = p.transpose(-1, -2).contiguous() @ do32
    dk_h = scale * (ds.transpose(-1, -2).contiguous() @ q32)
    dv = dv_h.reshape(b, hkv, grp, n, dd).sum(2)
    dk = dk_h.reshape(b, hkv, grp, n, dd).sum(2)
    return dq, dk, dv


def packed_layout(total: int, lo: int, hi: int, seed: int) -> list[int]:
    """Document lengths drawn uniform in [lo, hi] from `seed` until `total` is filled (last one
    truncated) -- the packed-attention workload (16384 tokens, lengths in [64, 2048], seed 0)."""
    import random

    rng = random.Random(seed)
    lens, used = [], 0
    while used < total:
        n = min(rng.randint(lo, hi), total - used)
        lens.append(n)
        used += n
    return lens


def segments_from_lengths(lengths: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
    """Gapless contiguous ascending seg_id and per-position seg_start (attention/segments.py:9-19)."""
    seg_id, seg_start, pos = [], [], 0
    for i, n in enumerate(lengths):
        seg_id += [i] * n
        seg_start += [pos] * n
        pos += n
    return torch.tensor(seg_id, dtype=torch.int32), torch.tensor(seg_start, dtype=torch.int32)
