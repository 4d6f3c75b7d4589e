"""4-bit affine group quantization in the MLX layout, on torch tensors (any device).

Layout (the one the reference's QuantizedHead carries, core/loss.py:36-41, and its kernel decodes,
core/kernel/source.py:193-208): w_q uint32 words [V][D/8] with 8 nibbles per word, first element in
the least-significant bits; scales and biases [V][D/64] in the head dtype; w = scale * q + bias.
torch has no uint32 tensor arithmetic on every backend, so words are carried as int32 bit patterns.
"""
from __future__ import annotations

import torch

from mlx_train_perf.errors import UnsupportedHeadError


def quantize(w: torch.Tensor, *, group_size: int = 64, bits: int = 4) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(V, D) -> (w_q int32 (V, D/8), scales (V, D/g), biases (V, D/g)) in w's dtype.

    s = (max - min) / 15, beta = min, q = round((w - beta) / s) per group of `group_size`
    consecutive elements of a row (MLX affine mode, typings/mlx/core/__init__.pyi:3229-3246)."""
    if bits != 4:
        raise UnsupportedHeadError(f"only bits=4 is supported (got bits={bits})")
    v, d = w.shape
    if d % group_size or d % 8:
        raise UnsupportedHeadError(f"D={d} must be a multiple of group_size={group_size}")
    wf = w.to(torch.float32).reshape(v, d // group_size, group_size)
    hi = wf.amax(dim=-1)
    lo = wf.amin(dim=-1)
    scales = ((hi - lo) / 15.0).to(w.dtype)
    biases = lo.to(w.dtype)
    s = scales.to(torch.float32)
    s = torch.where(s == 0, torch.ones_like(s), s)
    q = torch.round((wf - biases.to(torch.float32)[..., None]) / s[..., None]).clamp_(0, 15)
    q = q.to(torch.int64).reshape(v, d // 8, 8)
    shifts = torch.arange(8, dtype=torch.int64, device=w.device) * 4
    words = (q << shifts).sum(dim=-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    return words.contiguous(), scales.contiguous(), biases.contiguous()


def dequantize(w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, group_size: int = 64,
               bits: int = 4, dtype: torch.dtype | None = None) -> torch.Tensor:
    """w = scale * q + bias, computed in fp32 and returned in `dtype` (default: the scales' dtype)."""
    if bits != 4:
        raise UnsupportedHeadError(f"only bits=4 is supported (got bits={bits})")
    words = w_q.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, dtype=torch.int64, device=w_q.device) * 4
    q = ((words[..., None] >> shifts) & 0xF).reshape(w_q.shape[0], -1).to(torch.float32)
    s = scales.to(torch.float32).repeat_interleave(group_size, dim=1)
    b = biases.to(torch.float32).repeat_interleave(group_size, dim=1)
    out = s * q + b
    return out.to(dtype or scales.dtype)
