"""PackedMask: the packed-sequence segment carrier (mirror of src/mlx_train_perf/attention/segments.py)."""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class PackedMask:
    """Block-diagonal-causal segment description for one packed batch.

    seg_id: int32 (B, L) -- contiguous ascending segment ids per input position, starting at 0 each
      row; the pad tail is the row's last segment (gapless: every position belongs to one segment).
    seg_start: int32 (B, L) -- row index where the position's segment begins (non-decreasing).
    """
    seg_id: torch.Tensor
    seg_start: torch.Tensor


def segment_allowed(seg_id: torch.Tensor) -> torch.Tensor:
    """(B, 1, N, N) bool: key j visible to query i iff same segment AND j <= i (segments.py:22-29)."""
    same = seg_id[:, None, :, None] == seg_id[:, None, None, :]
    n = seg_id.shape[-1]
    causal = torch.tril(torch.ones(n, n, dtype=torch.bool, device=seg_id.device))[None, None]
    return same & causal
