"""Pins for the LCE oracle (oracle/lce.py) on the CPU.

Each check is chosen so that a plausible mistake (a dropped term, wrong sign or index, transposed
operand) fails it: hand-computed KATs (reference tests/test_naive.py:9-19), torch autograd of the
closed-form forward, central finite differences, chunk-boundary independence
(tests/test_chunked.py:95-99), and the softmax-minus-onehot row invariant. Planted mistakes are
applied to a copy of the oracle's formula to show the checks discriminate.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import lce as olce
from tests._inputs import lce_inputs


def test_hand_computed_two_rows():
    # D=2, V=3: logits row0 = [1, 0, -1], target 0; row1 = [0, 0, 0], target 1.
    h = torch.tensor([[1.0, 0.0], [0.0, 1.0]])
    w = torch.tensor([[1.0, 0.0], [0.0, 0.0], [-1.0, 0.0]])
    t = torch.tensor([0, 1])
    nll = olce.naive_linear_ce(h, w, t, dtype=torch.float64)
    assert abs(nll[0].item() - (math.log(math.e + 1 + math.exp(-1)) - 1.0)) < 1e-12
    assert abs(nll[1].item() - math.log(3.0)) < 1e-12
    nll2, lse, tgt = olce.forward(h, w, t, chunk=2)
    assert torch.allclose(nll2, nll) and abs(tgt[0].item() - 1.0) < 1e-12 and tgt[1].item() == 0.0


def test_streamed_equals_naive_and_chunk_independent():
    h, w, t = lce_inputs(33, 40, 517, seed=1, ignore_frac=0.0)
    ref = olce.naive_linear_ce(h, w, t, dtype=torch.float64)
    for chunk in (1, 7, 64, 517, 10_000):
        nll, lse, tgt = olce.forward(h, w, t, chunk=chunk)
        assert torch.allclose(nll, ref, atol=1e-12, rtol=0)
    logits = h.double() @ w.double().T
    assert (lse >= logits.max(dim=1).values - 1e-12).all()
    assert (nll >= 0).all()


def test_ignore_index_rows():
    h, w, t = lce_inputs(50, 16, 100, seed=2, ignore_frac=0.2)
    nll, lse, tgt = olce.forward(h, w, t)
    ign = t == -100
    assert ign.sum() == 10
    assert (nll[ign] == 0).all() and (tgt[ign] == 0).all() and torch.isfinite(lse[ign]).all()
    dh = olce.backward(h, w, t, lse, torch.ones(50), dtype=torch.float64)
    assert (dh[ign] == 0).all() and (dh[~ign].abs().sum(dim=1) > 0).all()


def _autograd_dh(h, w, t, ct):
    hh = h.double().clone().requires_grad_(True)
    nll = olce.naive_linear_ce(hh, w, t, dtype=torch.float64)
    (nll * ct.double()).sum().backward()
    return hh.grad


def test_backward_matches_autograd():
    h, w, t = lce_inputs(24, 32, 300, seed=3, ignore_frac=0.0)
    ct = torch.rand(24, generator=torch.Generator().manual_seed(0)) + 0.5
    _, lse, _ = olce.forward(h, w, t)
    dh = olce.backward(h, w, t, lse, ct, round_g_bf16=False, chunk=77, dtype=torch.float64)
    assert torch.allclose(dh, _autograd_dh(h, w, t, ct), atol=1e-12, rtol=1e-10)


def test_backward_finite_differences():
    g = torch.Generator().manual_seed(4)
    h = torch.randn(3, 5, generator=g, dtype=torch.float64)
    w = torch.randn(7, 5, generator=g, dtype=torch.float64)
    t = torch.tensor([0, 6, 3])
    _, lse, _ = olce.forward(h, w, t)
    dh = olce.backward(h, w, t, lse, torch.ones(3, dtype=torch.float64), round_g_bf16=False, dtype=torch.float64)
    eps = 1e-6
    for i in range(3):
        for j in range(5):
            hp, hm = h.clone(), h.clone()
            hp[i, j] += eps
            hm[i, j] -= eps
            fd = (olce.naive_linear_ce(hp, w, t, torch.float64).sum() - olce.naive_linear_ce(hm, w, t, torch.float64).sum()) / (2 * eps)
            assert abs(fd.item() - dh[i, j].item()) < 1e-7


def test_softmax_minus_onehot_rows_sum_to_zero():
    h, w, t = lce_inputs(10, 8, 50, seed=5, ignore_frac=0.0)
    _, lse, _ = olce.forward(h, w, t)
    logits = h.double() @ w.double().T
    p = torch.exp(logits - lse[:, None])
    onehot = torch.nn.functional.one_hot(t, 50).double()
    assert (p - onehot).sum(dim=1).abs().max() < 1e-12


@pytest.mark.parametrize("mistake", ["drop_onehot", "wrong_sign", "transpose_index"])
def test_planted_mistakes_fail_autograd_pin(mistake):
    """A wrong backward formula must not pass the autograd pin used above."""
    h, w, t = lce_inputs(12, 16, 40, seed=6, ignore_frac=0.0)
    ct = torch.ones(12, dtype=torch.float64)
    _, lse, _ = olce.forward(h, w, t)
    hd, wd = h.double(), w.double()
    p = torch.exp(hd @ wd.T - lse[:, None])
    onehot = torch.nn.functional.one_hot(t, 40).double()
    if mistake == "drop_onehot":
        g = p
    elif mistake == "wrong_sign":
        g = onehot - p
    else:
        g = (p - onehot).roll(1, dims=1)
    bad = g @ wd
    assert not torch.allclose(bad, _autograd_dh(h, w, t, ct), atol=1e-6)


def _rne_bf16_bits(x: torch.Tensor) -> torch.Tensor:
    """bf16 round-to-nearest-even of fp32 values by integer arithmetic on their bits (add 0x7FFF plus
    the lowest kept bit, clear the low 16 bits): independent of torch's bf16 cast. Finite inputs only."""
    b = x.to(torch.float32).view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return (b - ((b >> 31) << 32)).to(torch.int32).view(torch.float32)


def test_bf16_round_known_answers():
    """olce._bf16_round: bf16 keeps 8 significant bits and rounds half to even (not fp16's 11 bits,
    not truncation, not the identity)."""
    x = torch.tensor([1.0, 1 + 2**-8, 1 + 3 * 2**-9, 1 + 2**-9, 1 + 2**-7 + 2**-8, -(1 + 3 * 2**-9), 3.0e-5 * (1 + 2**-9),
                      65504.0 * 4, 2**-130], dtype=torch.float32)
    want = torch.tensor([1.0, 1.0, 1 + 2**-7, 1.0, 1 + 2**-6, -(1 + 2**-7), 3.0e-5, 2.0**18, 2**-130],
                        dtype=torch.float32)
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties go to the even mantissa (1.0), and
    # 1 + 2^-7 + 2^-8 (odd mantissa, halfway) goes up to 1 + 2^-6; 262016 = 2^18 - 128 needs 11
    # significant bits and rounds up into the next binade
    want[6] = _rne_bf16_bits(x[6:7])[0]
    got = olce._bf16_round(x)
    assert torch.equal(got, want), (got, want)
    assert torch.equal(got, _rne_bf16_bits(x))
    assert not torch.equal(got, x.half().float())   # fp16 would keep 1 + 2^-9


def test_bf16_round_matches_integer_rne():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(20000, generator=g) * torch.exp(torch.randn(20000, generator=g) * 8)
    got = olce._bf16_round(x)
    assert torch.equal(got, _rne_bf16_bits(x))
    assert (got != x).float().mean() > 0.99   # the rounding is visible on almost every random value


def test_backward_rounds_g_to_bf16():
    """backward(round_g_bf16=True) is the product of the bf16-RNE-rounded g (chunked.py:84-86): equal
    to g rounded by the integer method, and far from the unrounded and fp16-rounded products."""
    h, w, t = lce_inputs(24, 32, 300, seed=9)
    _, lse, _ = olce.forward(h, w, t, dtype=torch.float32)
    ct = torch.full((24,), 1.0 / 24)
    got = olce.backward(h, w, t, lse, ct, round_g_bf16=True, dtype=torch.float32, chunk=128)
    y = t.long()
    ctm = torch.where(y == -100, 0.0, ct)
    p = torch.exp(h.float() @ w.float().T - lse.float()[:, None])
    g = (p - torch.nn.functional.one_hot(y.clamp(min=0), 300).float() * (y >= 0).float()[:, None]) * ctm[:, None]
    want = _rne_bf16_bits(g) @ w.float()
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-7)
    unrounded = olce.backward(h, w, t, lse, ct, round_g_bf16=False, dtype=torch.float32, chunk=128)
    f16 = g.half().float() @ w.float()
    for other in (unrounded, f16):
        assert float((got - other).abs().max()) > 20 * float((got - want).abs().max()) + 1e-7


def test_bf16_rounding_of_g_is_small():
    h, w, t = lce_inputs(40, 64, 500, seed=7)
    _, lse, _ = olce.forward(h, w, t)
    ct = torch.ones(40)
    a = olce.backward(h, w, t, lse, ct, round_g_bf16=True, dtype=torch.float64)
    b = olce.backward(h, w, t, lse, ct, round_g_bf16=False, dtype=torch.float64)
    assert float((a - b).norm() / b.norm()) < 5e-3


def test_dw_matches_autograd_of_naive():
    h, w, t = lce_inputs(20, 16, 90, seed=11, ignore_frac=0.1)
    ct = torch.rand(20, generator=torch.Generator().manual_seed(3)) + 0.5
    _, lse, _ = olce.forward(h, w, t)
    dw = olce.backward_dw(h, w, t, lse, ct, round_g_bf16=False, chunk=33)
    ww = w.double().clone().requires_grad_(True)
    safe = torch.where(t == -100, torch.zeros_like(t), t)
    nll = olce.naive_linear_ce(h.double(), ww, safe, dtype=torch.float64)
    (nll * torch.where(t == -100, 0.0, ct.double())).sum().backward()
    assert torch.allclose(dw, ww.grad, atol=1e-12)


def test_reduce_mean_hand_computed():
    """reduce_mean: sum of the non-ignored rows over their count, by hand. Rows 1 and 3 are ignored;
    the kept rows hold 1.5, 4.0 and 0.5, so the mean is 6.0 / 3 = 2.0. A version that divided by all
    rows (1.2 with the ignored rows' 0 nll, 2.4 if they kept their values) or summed the ignored rows
    (12.0 / 3) fails; all ignored gives 0, not a division by zero."""
    nll = torch.tensor([1.5, 7.0, 4.0, -1.0, 0.5], dtype=torch.float64)
    t = torch.tensor([3, -100, 0, -100, 9])
    assert olce.reduce_mean(nll, t).item() == 2.0
    assert olce.reduce_mean(nll, t, ignore_index=9).item() == (1.5 + 7.0 + 4.0 - 1.0) / 4
    assert olce.reduce_mean(nll, torch.full((5,), -100)).item() == 0.0
    # it is the public reduction="mean" of the forward's per-row nll (ignored rows excluded)
    from mlx_train_perf import DenseHead, linear_cross_entropy

    h, w, tt = lce_inputs(40, 16, 50, seed=6, ignore_frac=0.25)
    got = linear_cross_entropy(h.float(), DenseHead(weight=w.float()), tt, impl="naive", reduction="mean")
    onll, _, _ = olce.forward(h, w, tt)
    assert abs(got.item() - olce.reduce_mean(onll, tt).item()) < 1e-6
