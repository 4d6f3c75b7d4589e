"""Pins for the affine 4-bit layout restatement (oracle/quant.py) and the product quantizer.

The nibble-order KAT mirrors the reference's tests/test_quant_layout.py:5-16 (positions crossing
nibble and word boundaries); the formula is the documented one
(typings/mlx/core/__init__.pyi:3229-3246, 3298-3302).
"""
from __future__ import annotations

import torch

from oracle import quant as oq


def _w(v=8, d=128, seed=17):
    return torch.randn(v, d, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def test_shapes_and_low_nibble_first_order():
    w = _w(8, 64)
    w_q, scales, biases = oq.quantize_affine(w.float())
    assert w_q.shape == (8, 8) and scales.shape == (8, 1) and biases.shape == (8, 1)
    w_dq = oq.dequantize_affine(w_q, scales, biases)
    for k in (0, 1, 7, 8, 63):
        packed = int(w_q[0, k // 8].item()) & 0xFFFFFFFF
        nib = (packed >> (4 * (k % 8))) & 0xF
        manual = float(scales[0, 0].float()) * nib + float(biases[0, 0].float())
        assert abs(manual - float(w_dq[0, k])) < 1e-6


def test_roundtrip_error_within_half_step():
    w = _w(16, 256).float()
    w_q, s, b = oq.quantize_affine(w)
    w_dq = oq.dequantize_affine(w_q, s, b)
    step = s.float().repeat_interleave(64, dim=1)
    # half a quantization step plus the bf16 rounding of scale/bias
    assert ((w_dq - w).abs() <= 0.5 * step + 2e-2 * w.abs().max()).all()
    codes = oq.unpack_nibbles(w_q)
    assert codes.min() >= 0 and codes.max() <= 15


def test_extremes_map_to_0_and_15():
    w = torch.zeros(1, 64)
    w[0, 5], w[0, 9] = -1.0, 2.0
    w_q, s, b = oq.quantize_affine(w, scale_dtype=torch.float32)
    codes = oq.unpack_nibbles(w_q)[0]
    assert codes[5] == 0 and codes[9] == 15
    assert abs(float(s[0, 0]) - 3.0 / 15) < 1e-7 and float(b[0, 0]) == -1.0


def test_product_quantizer_matches_oracle_bitwise():
    from mlx_train_perf.core.quant import dequantize, quantize

    w = _w(32, 192)
    a = quantize(w)
    b = oq.quantize_affine(w.float(), scale_dtype=torch.bfloat16)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert torch.equal(dequantize(*a, dtype=torch.float32), oq.dequantize_affine(*b))
