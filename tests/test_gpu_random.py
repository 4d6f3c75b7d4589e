"""GPU parity over seeded random shapes (the shapes are fixed by the seed, so every run checks the
same cases): LCE forward and dL/dH for dense and 4-bit heads (and dL/dW for a trainable head), and
attention forward and gradients with causal, non-causal and packed masks, against the CPU oracle,
at the same tolerances as the fixed-shape tests (per-token NLL 2e-3 relative, 8e-3 absolute for
the 4-bit head; gradients and O 1e-2 relative-L2; L 2e-3)."""
from __future__ import annotations

import math
import random

import pytest
import torch

from oracle import attention as oatt
from oracle import lce as olce
from oracle import quant as oquant
from tests._inputs import attn_inputs, lce_inputs, rel_l2
from tests.test_gpu_attention import _run_kernel, _segs

pytestmark = pytest.mark.gpu

IGN = -100
_R = random.Random(2026)
LCE_CASES = []
for _ in range(10):
    _n = _R.choice([_R.randint(1, 40), _R.randint(41, 700)])
    _d = _R.choice([64, 96, 128, 192, 200, 256, 320, 448, 512])
    _v = _R.choice([_R.randint(1, 300), _R.randint(301, 6000)])
    LCE_CASES.append((_n, _d, _v))
ATTN_CASES = []
for _ in range(10):
    _hkv, _g = _R.choice([1, 2, 4]), _R.choice([1, 2, 3, 4])
    ATTN_CASES.append((_R.randint(1, 2), _hkv * _g, _hkv, _R.randint(1, 700), _R.choice([64, 96, 128])))
NONCAUSAL_CASES = []
for _ in range(5):
    _hkv, _g = _R.choice([1, 2]), _R.choice([1, 2, 4])
    NONCAUSAL_CASES.append((_R.randint(1, 2), _hkv * _g, _hkv, _R.randint(1, 500), _R.choice([64, 96, 128])))
DW_CASES = [(_R.randint(1, 600), _R.choice([64, 128, 200, 256, 384]), _R.randint(2, 4000)) for _ in range(5)]
PACKED_CASES = []
for _ in range(6):
    _lens = [_R.randint(1, 200) for _ in range(_R.randint(1, 6))]
    _hkv, _g = _R.choice([1, 2]), _R.choice([1, 2, 4])
    PACKED_CASES.append((_lens, _hkv * _g, _hkv, _R.choice([64, 96, 128])))


# "default": the loss layer's head modes (a cached transposed copy for a frozen dense head, staged
# chunks for 4-bit and trainable heads, the staged 4-bit forward); "reads": no copy and no staging,
# so the dH products (and dW) read the head through LDS transpose reads, and a 4-bit head is
# dequantized in registers in every product.
MODES = ["default", "reads"]


def _set_mode(monkeypatch, mode):
    monkeypatch.delenv("MTP_LCE_TRANSPOSED_HEAD", raising=False)
    monkeypatch.delenv("MTP_LCE_STAGE_HEAD", raising=False)
    if mode == "reads":
        monkeypatch.setenv("MTP_LCE_TRANSPOSED_HEAD", "0")
        monkeypatch.setenv("MTP_LCE_STAGE_HEAD", "0")


def _lce_kernel(h, w, t, wq=None, sc=None, bi=None):
    from mlx_train_perf.core.loss import DenseHead, QuantizedHead, kernel_forward_parts

    hd = h.cuda().requires_grad_(True)
    head = (DenseHead(weight=w.cuda(), trainable=False) if wq is None
            else QuantizedHead(w_q=wq.cuda(), scales=sc.cuda(), biases=bi.cuda()))
    nll, lse, _ = kernel_forward_parts(hd, head, t.cuda(), ignore_index=IGN)
    return hd, nll, lse


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize(("n", "d", "v"), LCE_CASES)
def test_lce_random_dense(n, d, v, mode, monkeypatch):
    print(f"[lce random dense] n={n} d={d} v={v} mode={mode}", flush=True)
    _set_mode(monkeypatch, mode)
    h, w, t = lce_inputs(n, d, v, seed=n * 31 + d + v)
    hd, nll, lse = _lce_kernel(h, w, t)
    onll, olse, _ = olce.forward(h, w, t, ignore_index=IGN)
    assert ((nll.detach().cpu().double() - onll).abs() <= 2e-3 * onll.abs() + 1e-4).all()
    assert (lse.cpu().double() - olse).abs().max() <= 2e-3 * max(1.0, olse.abs().max().item())
    ct = torch.rand(n, generator=torch.Generator().manual_seed(n)) + 0.5
    nll.backward(ct.cuda())
    odh = olce.backward(h, w, t, olse, ct, ignore_index=IGN, round_g_bf16=True, dtype=torch.float64)
    if odh.abs().max() == 0:  # one class, or every row ignored: dL/dH is exactly 0
        assert hd.grad.abs().max() <= 1e-3
    else:
        assert rel_l2(hd.grad.cpu(), odh) <= 1e-2


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize(("n", "d", "v"), [c for c in LCE_CASES if c[1] % 64 == 0])
def test_lce_random_quantized(n, d, v, mode, monkeypatch):
    print(f"[lce random q4] n={n} d={d} v={v} mode={mode}", flush=True)
    _set_mode(monkeypatch, mode)
    h, w, t = lce_inputs(n, d, v, seed=n * 17 + d + v, w_std=0.05)
    wq, sc, bi = oquant.quantize_affine(w.float(), group_size=64, scale_dtype=torch.bfloat16)
    wdq = oquant.dequantize_affine(wq, sc, bi, group_size=64, dtype=torch.float32)
    hd, nll, lse = _lce_kernel(h, None, t, wq, sc, bi)
    onll, olse, _ = olce.forward(h, wdq, t, ignore_index=IGN)
    assert (nll.detach().cpu().double() - onll).abs().max() <= 8e-3
    ct = torch.rand(n, generator=torch.Generator().manual_seed(n + 1)) + 0.5
    nll.backward(ct.cuda())
    odh = olce.backward(h, wdq, t, olse, ct, ignore_index=IGN, round_g_bf16=True, dtype=torch.float64)
    if odh.abs().max() == 0:
        assert hd.grad.abs().max() <= 1e-3
    else:
        assert rel_l2(hd.grad.cpu(), odh) <= 1e-2


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize(("n", "d", "v"), DW_CASES)
def test_lce_random_trainable_head(n, d, v, mode, monkeypatch):
    from mlx_train_perf.core.loss import DenseHead, kernel_forward_parts

    print(f"[lce random dw] n={n} d={d} v={v} mode={mode}", flush=True)
    _set_mode(monkeypatch, mode)
    h, w, t = lce_inputs(n, d, v, seed=n * 13 + d + v)
    hd = h.cuda().requires_grad_(True)
    wd = w.cuda().requires_grad_(True)
    nll, lse, _ = kernel_forward_parts(hd, DenseHead(weight=wd, trainable=True), t.cuda(), ignore_index=IGN)
    ct = torch.rand(n, generator=torch.Generator().manual_seed(n + 2)) + 0.5
    nll.backward(ct.cuda())
    _, olse, _ = olce.forward(h, w, t, ignore_index=IGN)
    odh = olce.backward(h, w, t, olse, ct, ignore_index=IGN, dtype=torch.float64)
    odw = olce.backward_dw(h, w, t, olse, ct, ignore_index=IGN)
    assert rel_l2(hd.grad.cpu(), odh) <= 1e-2
    assert rel_l2(wd.grad.cpu(), odw) <= 1e-2


def _check_attention(res, q, k, v, do, scale, seg_id=None, causal=True):
    o, lse, dq, dk, dv = res
    oo, ol = oatt.attention_forward(q, k, v, scale=scale, causal=causal, seg_id=seg_id, dtype=torch.float64)
    odq, odk, odv = oatt.attention_backward(q, k, v, oo, ol, do, scale=scale, causal=causal, seg_id=seg_id,
                                            dtype=torch.float64)
    assert rel_l2(o, oo) <= 1e-2 and (lse.double() - ol).abs().max() <= 2e-3
    for got, want in ((dq, odq), (dk, odk), (dv, odv)):
        assert torch.isfinite(got.float()).all()
        if want.abs().max() < 1e-9:  # every row sees only its own key (s = 1 or 1-token segments)
            assert got.abs().max() <= 1e-3
        else:
            assert rel_l2(got, want) <= 1e-2


@pytest.mark.parametrize("shape", ATTN_CASES)
def test_attention_random_causal(shape):
    b, hq, hkv, s, d = shape
    print(f"[attn random causal] {shape}", flush=True)
    q, k, v, do = attn_inputs(b, hq, hkv, s, d, seed=5 * s + d + hq)
    scale = 1.0 / math.sqrt(d)
    _check_attention(_run_kernel(q, k, v, do, scale), q, k, v, do, scale)


@pytest.mark.parametrize("shape", NONCAUSAL_CASES)
def test_attention_random_noncausal(shape):
    b, hq, hkv, s, d = shape
    print(f"[attn random non-causal] {shape}", flush=True)
    q, k, v, do = attn_inputs(b, hq, hkv, s, d, seed=11 * s + d + hq)
    scale = 1.0 / math.sqrt(d)
    _check_attention(_run_kernel(q, k, v, do, scale, causal=False), q, k, v, do, scale, causal=False)


@pytest.mark.parametrize(("lengths", "hq", "hkv", "d"), PACKED_CASES)
def test_attention_random_packed(lengths, hq, hkv, d):
    print(f"[attn random packed] {lengths} hq={hq} hkv={hkv} d={d}", flush=True)
    s = sum(lengths)
    q, k, v, do = attn_inputs(1, hq, hkv, s, d, seed=s + 7 * d + hq)
    scale = 1.0 / math.sqrt(d)
    seg = _segs(lengths)
    _check_attention(_run_kernel(q, k, v, do, scale, seg=seg), q, k, v, do, scale, seg_id=seg[0])
