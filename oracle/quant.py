"""CPU restatement of MLX's affine group quantization (test infrastructure only).

The formula is the one the reference's vendored stubs document
(typings/mlx/core/__init__.pyi:3229-3246 quantize, :3298-3302 dequantize):
  alpha = max_i w_i, beta = min_i w_i over a group of g consecutive elements of a row,
  s = (alpha - beta) / (2^b - 1), q_i = round((w_i - beta) / s), w_i ~= s * q_i + beta,
with 32 // b values packed per uint32 from the least-significant bits up (first element in
bits 0-3 for b = 4). The reference kernel decodes exactly this layout
(core/kernel/source.py:193-208: nib = (wq[k >> 3] >> 4 (k & 7)) & 0xF, w = sc[g] * nib + bi[g]).

Parity does not depend on MLX's own rounding rules: kernel and oracle both dequantize the same
packed tensors (the "fp32-head lock" convention of tests/test_kernel_quant_parity.py:74-97).
"""
from __future__ import annotations

import torch


def quantize_affine(w: torch.Tensor, group_size: int = 64, bits: int = 4,
                    scale_dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """w (V, D) -> (w_q int32 bit patterns of uint32 words (V, D*bits/32), scales (V, D/g), biases (V, D/g)).

    Scales and biases are rounded to `scale_dtype` (the head's dtype, as in MLX) and the codes are
    computed against the rounded values, so dequantize(quantize(w)) uses exactly the stored
    parameters."""
    if bits != 4:
        raise ValueError("only 4-bit packing is restated here")
    v, d = w.shape
    if d % group_size:
        raise ValueError("D must be a multiple of group_size")
    wf = w.to(torch.float32).reshape(v, d // group_size, group_size)
    hi = wf.amax(dim=-1)
    lo = wf.amin(dim=-1)
    scales = ((hi - lo) / (2 ** bits - 1)).to(scale_dtype)
    biases = lo.to(scale_dtype)
    s = scales.to(torch.float32)
    s_safe = torch.where(s == 0, torch.ones_like(s), s)
    q = torch.round((wf - biases.to(torch.float32)[..., None]) / s_safe[..., None]).clamp(0, 2 ** bits - 1)
    q = q.to(torch.int64).reshape(v, d // 8, 8)
    shifts = torch.arange(8, dtype=torch.int64, device=w.device) * 4
    words = (q << shifts).sum(dim=-1)  # < 2^32
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    return words, scales, biases


def unpack_nibbles(w_q: torch.Tensor) -> torch.Tensor:
    """(V, D/8) uint32 words (as int32 bit patterns) -> (V, D) codes in [0, 15], low nibble first."""
    words = w_q.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, dtype=torch.int64, device=w_q.device) * 4
    return ((words[..., None] >> shifts) & 0xF).reshape(w_q.shape[0], -1)


def dequantize_affine(w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = 64,
                      dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """w = s * q + beta computed in `dtype` (fp32 by default: the reference's fp32-head lock)."""
    q = unpack_nibbles(w_q).to(dtype)
    v, d = q.shape
    s = scales.to(dtype).repeat_interleave(group_size, dim=1)
    b = biases.to(dtype).repeat_interleave(group_size, dim=1)
    return s * q + b
