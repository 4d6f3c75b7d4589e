"""Public API on the CPU: typed validation errors (reference tests/test_loss_api.py:117-210,
tests/test_attention_api.py), impl resolution without silent fallback, and the explicit torch impls
(`naive`, `chunked`, attention `reference`) against the oracle."""
from __future__ import annotations

import math

import pytest
import torch

from mlx_train_perf import DenseHead, QuantizedHead, linear_cross_entropy, resolve_impl, tied_head
from mlx_train_perf.attention import PackedMask, flash_attention, resolve_attention_impl
from mlx_train_perf.core import chunked as mchunked
from mlx_train_perf.core import loss as L
from mlx_train_perf.errors import (
    AttentionInputError,
    LossInputError,
    UnsupportedAttentionError,
    UnsupportedHeadError,
)
from oracle import attention as oa
from oracle import lce as olce
from oracle import quant as oq
from tests._inputs import lce_inputs


def _dense(v=50, d=16, trainable=False, dtype=torch.float32, seed=0):
    w = torch.randn(v, d, generator=torch.Generator().manual_seed(seed)).to(dtype)
    return DenseHead(weight=w, trainable=trainable)


def test_loss_input_validation():
    h = torch.randn(4, 16)
    t = torch.tensor([1, 2, 3, 4])
    head = _dense()
    with pytest.raises(LossInputError):
        linear_cross_entropy(h, head, t, reduction="avg")
    with pytest.raises(LossInputError):
        linear_cross_entropy(h[None, None], head, t)
    with pytest.raises(LossInputError):
        linear_cross_entropy(h, head, t[:3])
    with pytest.raises(LossInputError):
        linear_cross_entropy(h, head, t.float())
    with pytest.raises(LossInputError):
        linear_cross_entropy(h[:, :8], head, t)
    with pytest.raises(LossInputError):
        linear_cross_entropy(h.to(torch.bfloat16), head, t)
    with pytest.raises(LossInputError):
        linear_cross_entropy(h, head, torch.tensor([0, 1, 2, 50]), impl="naive")
    with pytest.raises(LossInputError):
        linear_cross_entropy(h, head, t, impl="fast")
    with pytest.raises(LossInputError):
        resolve_impl(head=head, dtype=torch.float32, n=0)


def test_kernel_gate_refusals_are_typed():
    bf = torch.bfloat16
    with pytest.raises(UnsupportedHeadError, match="fp32/bf16"):  # fp16 hidden: the kernels take fp32 or bf16
        resolve_impl(head=_dense(dtype=torch.float16), dtype=torch.float16, n=8)
    L._require_kernel_supported(head=_dense(), dtype=torch.float32)          # fp32 passes the dtype gate
    L._require_kernel_supported(head=_dense(d=12, dtype=bf), dtype=torch.float32)   # no d % 8 for fp32
    with pytest.raises(UnsupportedHeadError, match="multiple of 8"):
        L._require_kernel_supported(head=_dense(d=12, dtype=bf), dtype=bf)
    wq, sc, bi = oq.quantize_affine(torch.randn(10, 64))
    with pytest.raises(UnsupportedHeadError):
        resolve_impl(head=QuantizedHead(w_q=wq, scales=sc, biases=bi, bits=8), dtype=bf, n=8)
    with pytest.raises(UnsupportedHeadError):
        resolve_impl(head=QuantizedHead(w_q=wq, scales=sc, biases=bi, group_size=32), dtype=bf, n=8)
    if not torch.cuda.is_available():
        with pytest.raises(UnsupportedHeadError):  # no GPU: refused, never a CPU fallback
            resolve_impl(head=_dense(dtype=bf), dtype=bf, n=8, impl="auto")
    assert resolve_impl(head=_dense(), dtype=torch.float32, n=8, impl="chunked").impl == "chunked"
    assert tied_head(torch.zeros(3, 4)).trainable is False


@pytest.mark.parametrize("impl", ["naive", "chunked"])
def test_explicit_torch_impls_match_oracle(impl):
    h, w, t = lce_inputs(40, 32, 300, seed=1)
    h32, w32 = h.float(), w.float()
    hh = h32.clone().requires_grad_(True)
    ww = w32.clone().requires_grad_(True)
    loss = linear_cross_entropy(hh, DenseHead(weight=ww, trainable=True), t, impl=impl, chunk_size=64)
    loss.backward()
    onll, olse, _ = olce.forward(h32, w32, t)
    valid = t != -100
    assert abs(loss.item() - (onll[valid].sum() / valid.sum()).item()) < 1e-5
    odh = olce.backward(h32, w32, t, olse, valid.double() / valid.sum(), round_g_bf16=False, dtype=torch.float64)
    assert torch.allclose(hh.grad.double(), odh, atol=1e-6)
    assert ww.grad is not None and torch.isfinite(ww.grad).all()


def test_chunked_quantized_matches_dequantized_oracle():
    h, w, t = lce_inputs(20, 64, 200, seed=2, w_std=0.05)
    wq, sc, bi = oq.quantize_affine(w.float(), scale_dtype=torch.float32)
    head = QuantizedHead(w_q=wq, scales=sc, biases=bi)
    hh = h.float().clone().requires_grad_(True)
    nll = linear_cross_entropy(hh, head, t, impl="chunked", chunk_size=64, reduction="none")
    nll.sum().backward()
    wdq = oq.dequantize_affine(wq, sc, bi)
    onll, olse, _ = olce.forward(h.float(), wdq, t)
    assert torch.allclose(nll.double(), onll, atol=1e-5)
    odh = olce.backward(h.float(), wdq, t, olse, torch.ones(20), round_g_bf16=False, dtype=torch.float64)
    assert torch.allclose(hh.grad.double(), odh, atol=1e-5)
    assert mchunked.VJP_CALLS.get("quantized", 0) >= 1


def test_reductions_and_3d_input():
    h, w, t = lce_inputs(24, 16, 90, seed=3)
    head = DenseHead(weight=w.float(), trainable=False)
    none = linear_cross_entropy(h.float().reshape(4, 6, 16), head, t.reshape(4, 6), impl="naive", reduction="none")
    assert none.shape == (4, 6)
    s = linear_cross_entropy(h.float(), head, t, impl="naive", reduction="sum")
    assert torch.allclose(s, none.sum())
    assert (none.reshape(-1)[t == -100] == 0).all()


def _attn(b=1, hq=4, hkv=2, n=12, d=8, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, hq, n, d, generator=g).to(dtype), torch.randn(b, hkv, n, d, generator=g).to(dtype),
            torch.randn(b, hkv, n, d, generator=g).to(dtype))


def test_attention_validation():
    q, k, v = _attn()
    with pytest.raises(AttentionInputError):
        flash_attention(q[0], k, v, scale=1.0)
    with pytest.raises(AttentionInputError):
        flash_attention(q, k[:, :1], v, scale=1.0)
    with pytest.raises(AttentionInputError):
        flash_attention(q[:, :3], k, v, scale=1.0)
    with pytest.raises(AttentionInputError):
        flash_attention(q, k[:, :, :5], v, scale=1.0)
    with pytest.raises(AttentionInputError):
        flash_attention(q, k, v, scale=1.0, impl="magic")
    pm = PackedMask(seg_id=torch.zeros(1, 12, dtype=torch.int32), seg_start=torch.zeros(1, 12, dtype=torch.int32))
    with pytest.raises(UnsupportedAttentionError):
        flash_attention(q, k, v, scale=1.0, causal=False, segments=pm)
    with pytest.raises(UnsupportedAttentionError, match="fp32/bf16"):  # fp16: the kernels take fp32 or bf16
        resolve_attention_impl(q.half(), k.half(), v.half(), impl="kernel")
    qb, kb, vb = _attn(d=80, dtype=torch.bfloat16)
    with pytest.raises(UnsupportedAttentionError):
        resolve_attention_impl(qb, kb, vb, impl="auto")
    qb, kb, vb = _attn(d=64, dtype=torch.bfloat16)
    if not torch.cuda.is_available():   # no GPU: refused, never a CPU fallback (causal or not)
        with pytest.raises(UnsupportedAttentionError):
            resolve_attention_impl(qb, kb, vb, impl="auto")
        with pytest.raises(UnsupportedAttentionError):
            resolve_attention_impl(qb, kb, vb, impl="kernel", causal=False)


@pytest.mark.parametrize("packed", [False, True])
def test_reference_impl_matches_oracle(packed):
    q, k, v = _attn(n=10, seed=4)
    seg = None
    sid = None
    if packed:
        sid, sst = oa.segments_from_lengths([4, 6])
        seg = PackedMask(seg_id=sid[None], seg_start=sst[None])
        sid = sid[None]
    qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
    o = flash_attention(qq, kk, vv, scale=0.35, impl="reference", segments=seg)
    do = torch.randn(o.shape, generator=torch.Generator().manual_seed(1))
    o.backward(do)
    oo, ol = oa.attention_forward(q, k, v, scale=0.35, seg_id=sid, dtype=torch.float64)
    grads = oa.attention_backward(q, k, v, oo, ol, do, scale=0.35, seg_id=sid, dtype=torch.float64)
    assert torch.allclose(o.double(), oo, atol=1e-5)
    for got, want in zip((qq.grad, kk.grad, vv.grad), grads):
        assert torch.allclose(got.double(), want, atol=1e-5)
    assert math.isfinite(float(o.detach().sum()))


def test_quantized_head_kernel_gate_checks_dtypes_and_shapes():
    """The kernels read w_q as 32-bit words and scales/biases as bf16 (V, D/64): other dtypes are
    refused by the kernel gate (naming impl='chunked'), wrong shapes by the input check (any impl)."""
    bf = torch.bfloat16
    wq, sc, bi = oq.quantize_affine(torch.randn(10, 64), scale_dtype=torch.float32)
    with pytest.raises(UnsupportedHeadError, match="chunked"):  # fp32 scales with bf16 hidden states
        resolve_impl(head=QuantizedHead(w_q=wq, scales=sc, biases=bi.to(bf)), dtype=bf, n=8)
    with pytest.raises(UnsupportedHeadError, match="chunked"):  # fp32 biases with bf16 hidden states
        resolve_impl(head=QuantizedHead(w_q=wq, scales=sc.to(bf), biases=bi), dtype=bf, n=8)
    # fp32 hidden states: the fp32 kernels take fp32 or bf16 scales and biases, not fp16
    L._require_kernel_supported(head=QuantizedHead(w_q=wq, scales=sc, biases=bi), dtype=torch.float32)
    L._require_kernel_supported(head=QuantizedHead(w_q=wq, scales=sc.to(bf), biases=bi.to(bf)), dtype=torch.float32)
    with pytest.raises(UnsupportedHeadError, match="chunked"):
        L._require_kernel_supported(head=QuantizedHead(w_q=wq, scales=sc.half(), biases=bi), dtype=torch.float32)
    with pytest.raises(UnsupportedHeadError, match="32-bit"):  # 64-bit words
        resolve_impl(head=QuantizedHead(w_q=wq.long(), scales=sc.to(bf), biases=bi.to(bf)), dtype=bf, n=8)
    h = torch.randn(4, 64).to(bf)
    t = torch.tensor([0, 1, 2, 3])
    for bad in (sc[:, :0], sc[:5], torch.cat([sc, sc], dim=1)):
        with pytest.raises(LossInputError, match="scales"):
            linear_cross_entropy(h, QuantizedHead(w_q=wq, scales=bad.to(bf), biases=bi.to(bf)), t, impl="chunked")
    with pytest.raises(LossInputError, match="biases"):
        linear_cross_entropy(h, QuantizedHead(w_q=wq, scales=sc.to(bf), biases=bi[:3].to(bf)), t, impl="chunked")


def test_kernel_path_requires_inputs_on_hidden_device(monkeypatch):
    """A targets / head tensor on another device than hidden is refused before any launch (a host
    pointer passed to a kernel would fault the GPU). Run on the CPU with the GPU gate stubbed out
    and hidden on the `meta` device standing in for the GPU."""
    from mlx_train_perf import _compat
    from mlx_train_perf.core import loss as L

    monkeypatch.setattr(_compat, "require_gpu_tensor", lambda t, error: None)
    h = torch.empty(4, 64, dtype=torch.bfloat16, device="meta")
    w = torch.empty(10, 64, dtype=torch.bfloat16, device="meta")
    t_meta = torch.empty(4, dtype=torch.int64, device="meta")
    with pytest.raises(LossInputError, match="targets"):
        L._require_same_device(h, DenseHead(weight=w), torch.zeros(4, dtype=torch.int64))
    with pytest.raises(LossInputError, match="head.weight"):
        L._require_same_device(h, DenseHead(weight=torch.zeros(10, 64, dtype=torch.bfloat16)), t_meta)
    wq, sc, bi = oq.quantize_affine(torch.randn(10, 64))
    qh = QuantizedHead(w_q=wq.to("meta"), scales=sc.to("meta"), biases=bi)
    with pytest.raises(LossInputError, match="head.biases"):
        L._require_same_device(h, qh, t_meta)
    L._require_same_device(h, DenseHead(weight=w), t_meta)  # all on one device: accepted


def test_attention_requires_one_device():
    q, k, v = _attn()
    with pytest.raises(AttentionInputError, match="one device"):
        flash_attention(q, k.to("meta"), v, scale=1.0, impl="reference")


@pytest.mark.parametrize(("sid", "sst", "what"), [
    ([[0, 0, 1, 1, 1]], [[0, 0, 2, 2, 2]], None),
    ([[0, 0, 0, 0, 0]], [[0, 0, 0, 0, 0]], None),
    ([[0, 1, 2, 3, 4]], [[0, 1, 2, 3, 4]], None),
    ([[1, 1, 2, 2, 2]], [[0, 0, 2, 2, 2]], "start at 0"),
    ([[0, 0, 2, 2, 2]], [[0, 0, 2, 2, 2]], "contiguous"),
    ([[0, 0, 1, 1, 0]], [[0, 0, 2, 2, 4]], "contiguous"),
    ([[0, 0, 1, 1, 1]], [[0, 0, 2, 2, 3]], "seg_start"),
    ([[0, 0, 1, 1, 1]], [[0, 0, 0, 0, 0]], "seg_start"),
    ([[0, 0, 1, 1, 1]], [[-1, 0, 2, 2, 2]], "seg_start"),
    ([[0, 0, 1, 1, 1], [0, 1, 1, 1, 1]], [[0, 0, 2, 2, 2], [0, 1, 1, 1, 2]], "seg_start"),
])
def test_packed_layout_contract(sid, sst, what):
    """layout_violation accepts exactly the PackedMask contract; flash_attention refuses a violating
    layout with AttentionInputError (the kernels mask by seg_start ranges, the oracle by seg_id, so
    the two agree only on valid layouts), and skips the check when asked to."""
    from mlx_train_perf.attention.segments import layout_violation

    sid_t = torch.tensor(sid, dtype=torch.int32)
    sst_t = torch.tensor(sst, dtype=torch.int32)
    got = layout_violation(sid_t, sst_t)
    if what is None:
        assert got is None
        return
    assert got is not None and what in got
    b = sid_t.shape[0]
    q, k, v = _attn(b=b, n=5)
    with pytest.raises(AttentionInputError, match="layout contract"):
        flash_attention(q, k, v, scale=1.0, impl="reference", segments=PackedMask(seg_id=sid_t, seg_start=sst_t))
    flash_attention(q, k, v, scale=1.0, impl="reference", segments=PackedMask(seg_id=sid_t, seg_start=sst_t),
                    validate_segments=False)


def test_packed_layout_check_runs_again_after_in_place_edit():
    from mlx_train_perf.attention import api

    sid, sst = oa.segments_from_lengths([2, 3])
    pm = PackedMask(seg_id=sid[None].clone(), seg_start=sst[None].clone())
    q, k, v = _attn(n=5)
    flash_attention(q, k, v, scale=1.0, impl="reference", segments=pm)
    assert api._layout_seen(pm)
    pm.seg_start[0, 4] = 3   # breaks the contract in place
    assert not api._layout_seen(pm)
    with pytest.raises(AttentionInputError):
        flash_attention(q, k, v, scale=1.0, impl="reference", segments=pm)
