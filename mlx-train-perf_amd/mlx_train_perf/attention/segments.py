"""Segment description of a packed batch (the reference's `PackedMask`,
src/mlx_train_perf/attention/segments.py:9-29), plus the checks of its layout contract."""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class PackedMask:
    """Which documents share one packed row, as two int32 (B, L) tensors.

    seg_id: the document number of each position. Numbers start at 0 in every row and go up by
      one at each document boundary; padding at the end of a row is one more document, so every
      position has a number.
    seg_start: the index of the first position of the document each position belongs to; it never
      decreases along a row.
    """
    seg_id: torch.Tensor
    seg_start: torch.Tensor


def segment_allowed(seg_id: torch.Tensor) -> torch.Tensor:
    """Visibility as a (B, 1, N, N) bool tensor: query i may attend key j when both positions carry
    the same document number and j does not come after i."""
    same = seg_id[:, None, :, None] == seg_id[:, None, None, :]
    n = seg_id.shape[-1]
    causal = torch.tril(torch.ones(n, n, dtype=torch.bool, device=seg_id.device))[None, None]
    return same & causal


def layout_violation(seg_id: torch.Tensor, seg_start: torch.Tensor) -> str | None:
    """None when (seg_id, seg_start) follows the packed-row contract, else what is wrong.

    The contract, per row: seg_id starts at 0 and each step along the row adds 0 or 1 to it; a
    position starts a document exactly where seg_id steps up (or at 0); seg_start[i] is that start
    for every position i. The kernels mask with seg_start ranges, so a layout off the contract would
    be masked differently from seg_id equality -- hence the check. One device pass, one host sync."""
    sid = seg_id.to(torch.int64)
    sst = seg_start.to(torch.int64)
    n = sid.shape[-1]
    pos = torch.arange(n, device=sid.device).expand_as(sid)
    step = torch.diff(sid, dim=-1)
    new_doc = torch.ones_like(sid, dtype=torch.bool)
    new_doc[:, 1:] = step == 1
    # the start of each position's document: the last index <= i where a document begins
    starts = torch.cummax(torch.where(new_doc, pos, torch.zeros_like(pos)), dim=-1).values
    checks = torch.stack([
        (sid[:, 0] != 0).any(),
        ((step != 0) & (step != 1)).any(),
        (sst != starts).any(),
    ]).cpu()
    if checks[0]:
        return "seg_id must start at 0 in every row"
    if checks[1]:
        return "seg_id must be contiguous and ascending (each step along a row adds 0 or 1)"
    if checks[2]:
        return "seg_start must hold the first position of each position's segment (as implied by seg_id)"
    return None
