"""The kernel paths under HIP graph capture (torch.cuda.graph): a loss step (forward and dL/dH
through the C-ABI, dense and 4-bit heads) and causal and packed GQA attention steps (forward, dQ and
dK/dV), captured once after warm-up on a side stream and replayed with new inputs copied into the
static tensors. Every replay is checked bitwise against an eager run on the same inputs, with eager work
on the device between the replays (a captured graph must not depend on state the eager work
changes). The library launches nothing but kernels on the caller's stream and needs no cleared
memory, so its launches are capture-safe; the Python layer allocates workspaces from torch, which
serves them from the graph's private pool."""
from __future__ import annotations

import pytest
import torch

from tests._inputs import attn_inputs, lce_inputs

pytestmark = pytest.mark.gpu


def _eager_work():
    # unrelated eager kernels between replays (a matmul and a multi-block reduction)
    a = torch.randn(512, 512, device="cuda")
    return float((a @ a).sum())


def _capture(fn, warmup=3):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


@pytest.mark.parametrize("kind", ["dense", "q4"])
def test_lce_step_replays_in_a_hip_graph(kind):
    from mlx_train_perf import DenseHead, QuantizedHead, linear_cross_entropy
    from oracle import quant as oquant

    print(f"[graph lce {kind}]", flush=True)
    n, d, v = 512, 256, 3000
    h0, w, t0 = lce_inputs(n, d, v, seed=1)
    if kind == "dense":
        head = DenseHead(weight=w.cuda(), trainable=False)
    else:
        wq, sc, bi = oquant.quantize_affine(w.float())
        head = QuantizedHead(w_q=wq.cuda(), scales=sc.cuda(), biases=bi.cuda())
    hs = h0.cuda().requires_grad_(True)
    ts = t0.cuda()
    ct = torch.full((n,), 1.0 / n, device="cuda")

    def step():
        hs.grad = None
        nll = linear_cross_entropy(hs, head, ts, reduction="none", validate_targets=False)
        nll.backward(ct)
        return nll

    g, nll_static = _capture(step)
    for rep in range(3):
        h1, _, t1 = lce_inputs(n, d, v, seed=10 + rep)
        with torch.no_grad():
            hs.copy_(h1.cuda())
        ts.copy_(t1.cuda())
        g.replay()
        torch.cuda.synchronize()
        got_nll, got_dh = nll_static.detach().clone(), hs.grad.detach().clone()
        _eager_work()
        he = h1.cuda().requires_grad_(True)
        nll_e = linear_cross_entropy(he, head, t1.cuda(), reduction="none", validate_targets=False)
        nll_e.backward(ct)
        torch.cuda.synchronize()
        assert torch.equal(got_nll, nll_e.detach()), f"replay {rep}: nll"
        assert torch.equal(got_dh, he.grad), f"replay {rep}: dH"


def test_attention_step_replays_in_a_hip_graph():
    from mlx_train_perf.attention import flash_attention

    print("[graph attention]", flush=True)
    b, hq, hkv, s, d = 1, 8, 2, 300, 128
    q0, k0, v0, do0 = attn_inputs(b, hq, hkv, s, d, seed=3)
    qs, ks, vs = (x.cuda().requires_grad_(True) for x in (q0, k0, v0))
    dos = do0.cuda()
    scale = d ** -0.5

    def step():
        for x in (qs, ks, vs):
            x.grad = None
        o = flash_attention(qs, ks, vs, scale=scale)
        o.backward(dos)
        return o

    g, o_static = _capture(step)
    for rep in range(3):
        q1, k1, v1, do1 = attn_inputs(b, hq, hkv, s, d, seed=20 + rep)
        with torch.no_grad():
            for dst, src in ((qs, q1), (ks, k1), (vs, v1)):
                dst.copy_(src.cuda())
        dos.copy_(do1.cuda())
        g.replay()
        torch.cuda.synchronize()
        got = [o_static.detach().clone()] + [x.grad.detach().clone() for x in (qs, ks, vs)]
        _eager_work()
        qe, ke, ve = (x.cuda().requires_grad_(True) for x in (q1, k1, v1))
        oe = flash_attention(qe, ke, ve, scale=scale)
        oe.backward(do1.cuda())
        torch.cuda.synchronize()
        for name, a, e in zip(("O", "dQ", "dK", "dV"), got, (oe.detach(), qe.grad, ke.grad, ve.grad)):
            assert torch.equal(a, e), f"replay {rep}: {name}"


def test_packed_attention_step_replays_in_a_hip_graph():
    """Packed rows: the backward's work-order sort and segment-end table are kernels too. The layout
    check of a PackedMask runs on the host once per mask (during the warm-up), so the captured step
    holds no host synchronization; replays take new layouts copied into the same mask tensors."""
    from mlx_train_perf.attention import PackedMask, flash_attention
    from oracle import attention as oatt

    print("[graph attention packed]", flush=True)
    b, hq, hkv, d = 1, 8, 2, 128
    layouts = [[100, 37, 120, 43], [3, 297], [300], [64, 64, 64, 108]]
    s = sum(layouts[0])
    q0, k0, v0, do0 = attn_inputs(b, hq, hkv, s, d, seed=4)
    qs, ks, vs = (x.cuda().requires_grad_(True) for x in (q0, k0, v0))
    dos = do0.cuda()
    sid0, sst0 = oatt.segments_from_lengths(layouts[0])
    mask = PackedMask(seg_id=sid0[None].cuda().int().contiguous(), seg_start=sst0[None].cuda().int().contiguous())
    scale = d ** -0.5

    def step():
        for x in (qs, ks, vs):
            x.grad = None
        o = flash_attention(qs, ks, vs, scale=scale, segments=mask)
        o.backward(dos)
        return o

    g, o_static = _capture(step)
    for rep, lens in enumerate(layouts[1:]):
        assert sum(lens) == s
        q1, k1, v1, do1 = attn_inputs(b, hq, hkv, s, d, seed=30 + rep)
        sid1, sst1 = oatt.segments_from_lengths(lens)
        with torch.no_grad():
            for dst, src in ((qs, q1), (ks, k1), (vs, v1)):
                dst.copy_(src.cuda())
        dos.copy_(do1.cuda())
        mask.seg_id.copy_(sid1[None].cuda())
        mask.seg_start.copy_(sst1[None].cuda())
        g.replay()
        torch.cuda.synchronize()
        got = [o_static.detach().clone()] + [x.grad.detach().clone() for x in (qs, ks, vs)]
        _eager_work()
        qe, ke, ve = (x.cuda().requires_grad_(True) for x in (q1, k1, v1))
        m1 = PackedMask(seg_id=sid1[None].cuda().int().contiguous(), seg_start=sst1[None].cuda().int().contiguous())
        oe = flash_attention(qe, ke, ve, scale=scale, segments=m1)
        oe.backward(do1.cuda())
        torch.cuda.synchronize()
        for name, a, e in zip(("O", "dQ", "dK", "dV"), got, (oe.detach(), qe.grad, ke.grad, ve.grad)):
            assert torch.equal(a, e), f"replay {rep} ({lens}): {name}"
