"""GPU parity of the fp32 entry points (fp32 hidden states / q, k, v) against the fp64 oracle.

The reference kernels take fp32 as well as bf16 and pin fp32 tightly (max-abs):
- LCE forward nll 4e-6 (tests/test_kernel_parity.py:20,43: n <= 8192, d <= 64, w ~ 0.05 N(0,1));
  its stated fp32 ceiling is 1e-5, which BASELINE config 1 (d = 512, v = 32000) is held to here;
- LCE backward dL/dH 2e-6 (tests/test_kernel_backward.py:85);
- attention forward O and L 2e-6 (tests/test_attention_kernel_fwd.py:460-465), D 2e-5, dQ 5e-6,
  dK / dV 2.5e-5 (tests/test_attention_kernel_bwd.py:135,345,654), inputs ~ N(0, 1), n <= 257.
Those bars apply here at the same shapes and distributions. The oracle runs in fp64 on the GPU.
"""
from __future__ import annotations

import math
import random as _random

import pytest
import torch

from oracle import attention as oatt
from oracle import lce as olce
from oracle import quant as oquant
from tests._inputs import rel_l2

pytestmark = pytest.mark.gpu

IGN = -100


def _lce_fp32(h, head, t, ct, chunk=None):
    from mlx_train_perf.core.loss import kernel_forward_parts

    hd = h.cuda().requires_grad_(True)
    nll, lse, tgt = kernel_forward_parts(hd, head, t.cuda(), ignore_index=IGN, bwd_chunk=chunk)
    nll.backward(ct.cuda())
    torch.cuda.synchronize()
    return nll.detach().cpu().double(), lse.cpu().double(), tgt.cpu().double(), hd.grad.cpu().double()


@pytest.mark.parametrize(("n", "d", "v"), [(64, 32, 1000), (128, 64, 8192), (65, 33, 1027), (512, 64, 2048),
                                           (300, 200, 3000)])
def test_lce_fp32_reference_grid(n, d, v):
    """The reference's fp32 parity grid (tests/test_kernel_parity.py:11-17): forward nll within 4e-6,
    dL/dH within 2e-6 max-abs (cotangents of magnitude 0.1-2 with alternating signs,
    tests/test_kernel_backward.py:40-47)."""
    from mlx_train_perf import DenseHead

    print(f"[lce fp32 n={n} d={d} v={v}]", flush=True)
    g = torch.Generator().manual_seed(3)
    h = torch.randn(n, d, generator=g)
    w = torch.randn(v, d, generator=g) * 0.05
    t = torch.randint(0, v, (n,), generator=g)
    t[0], t[1], t[2] = 0, v - 1, min(256, v) - 1
    ct = torch.rand(n, generator=g) * 1.9 + 0.1
    ct = ct * torch.where(torch.arange(n) % 2 == 0, 1.0, -1.0)
    nll, lse, tgt, dh = _lce_fp32(h, DenseHead(weight=w.cuda(), trainable=False), t, ct)
    onll, olse, otgt = olce.forward(h.cuda(), w.cuda(), t.cuda(), dtype=torch.float64)
    odh = olce.backward(h.cuda(), w.cuda(), t.cuda(), olse, ct.cuda(), round_g_bf16=False, dtype=torch.float64)
    e_nll = float((nll - onll.cpu()).abs().max())
    e_dh = float((dh - odh.cpu()).abs().max())
    print(f"  nll max-abs {e_nll:.2e}, lse {float((lse - olse.cpu()).abs().max()):.2e}, dH max-abs {e_dh:.2e}",
          flush=True)
    assert e_nll < 4e-6 and e_dh < 2e-6
    assert float((tgt - otgt.cpu()).abs().max()) < 4e-6


def test_lce_fp32_config1():
    """BASELINE config 1 in fp32 on the kernel: N=1024, D=512, V=32000, H ~ N(0,1), W ~ N(0, 0.02^2),
    102 rows ignore_index; nll within 1e-5 max-abs (the reference's fp32 ceiling), the masked mean
    within 1e-6 relative, dL/dH of the mean within 1e-5 relative-L2 and ignored rows exactly 0; then a
    trainable head's dL/dW and a multi-chunk backward (128-column chunks)."""
    from mlx_train_perf import DenseHead, linear_cross_entropy

    print("[lce fp32 config 1]", flush=True)
    g = torch.Generator().manual_seed(0)
    n, d, v = 1024, 512, 32000
    h = torch.randn(n, d, generator=g)
    w = torch.randn(v, d, generator=g) * 0.02
    t = torch.randint(0, v, (n,), generator=g)
    t[torch.randperm(n, generator=g)[:102]] = IGN
    valid = t != IGN
    ct = valid.double() / valid.sum()
    hc, wc, tc = h.cuda(), w.cuda(), t.cuda()
    onll, olse, _ = olce.forward(hc, wc, tc, dtype=torch.float64)
    odh = olce.backward(hc, wc, tc, olse, ct.cuda(), round_g_bf16=False, dtype=torch.float64).cpu()

    hd = hc.clone().requires_grad_(True)
    loss = linear_cross_entropy(hd, DenseHead(weight=wc, trainable=False), tc, reduction="mean")
    loss.backward()
    oloss = float(olce.reduce_mean(onll, tc))
    assert abs(loss.item() - oloss) <= 1e-6 * abs(oloss), (loss.item(), oloss)
    nll = linear_cross_entropy(hc, DenseHead(weight=wc, trainable=False), tc, reduction="none").double().cpu()
    e_nll = float((nll - onll.cpu()).abs().max())
    r_dh = rel_l2(hd.grad.cpu(), odh)
    print(f"  nll max-abs {e_nll:.2e}, dH rel-L2 {r_dh:.2e}", flush=True)
    assert e_nll < 1e-5 and r_dh < 1e-5
    assert (hd.grad[~valid.cuda()] == 0).all()

    # trainable head: dL/dW (and the same dH) against the oracle's g^T h
    wd = wc.clone().requires_grad_(True)
    hd2 = hc.clone().requires_grad_(True)
    linear_cross_entropy(hd2, DenseHead(weight=wd, trainable=True), tc, reduction="mean").backward()
    odw = olce.backward_dw(hc, wc, tc, olse, ct.cuda(), round_g_bf16=False, dtype=torch.float64).cpu()
    r_dw = rel_l2(wd.grad.cpu(), odw)
    print(f"  dW rel-L2 {r_dw:.2e}", flush=True)
    assert r_dw < 1e-5 and rel_l2(hd2.grad.cpu(), odh) < 1e-5

    # 128-column vocab chunks: dH accumulated in fp32 over 250 chunks, dW per chunk
    wd3 = wc.clone().requires_grad_(True)
    hd3 = hc.clone().requires_grad_(True)
    linear_cross_entropy(hd3, DenseHead(weight=wd3, trainable=True), tc, reduction="mean", chunk_size=128).backward()
    assert rel_l2(hd3.grad.cpu(), odh) < 1e-5 and rel_l2(wd3.grad.cpu(), odw) < 1e-5

    # 4096-column chunks: each chunk's dH product splits its contraction (8 parts, 6 in the last
    # chunk) and the part sums accumulate into dH over 8 chunks
    hd4 = hc.clone().requires_grad_(True)
    linear_cross_entropy(hd4, DenseHead(weight=wc, trainable=False), tc, reduction="mean", chunk_size=4096).backward()
    r4 = rel_l2(hd4.grad.cpu(), odh)
    print(f"  dH rel-L2 with 4096-column chunks {r4:.2e}", flush=True)
    assert r4 < 1e-5


def test_lce_fp32_quantized_head():
    """A 4-bit head with fp32 hidden states: against the oracle on the head dequantized in fp64 (the
    reference's fp32-head convention, tests/test_kernel_quant_parity.py:74-97); scales stored as fp32
    or bf16."""
    from mlx_train_perf import QuantizedHead

    print("[lce fp32 4-bit head]", flush=True)
    g = torch.Generator().manual_seed(5)
    n, d, v = 200, 128, 3000
    h = torch.randn(n, d, generator=g)
    t = torch.randint(0, v, (n,), generator=g)
    t[:7] = IGN
    ct = torch.where(t == IGN, 0.0, 1.0 / n)
    for sdt in (torch.float32, torch.bfloat16):
        wq, sc, bi = oquant.quantize_affine(torch.randn(v, d, generator=g) * 0.05, scale_dtype=sdt)
        wdq = oquant.dequantize_affine(wq, sc, bi, dtype=torch.float64)
        head = QuantizedHead(w_q=wq.cuda(), scales=sc.cuda(), biases=bi.cuda())
        nll, _, _, dh = _lce_fp32(h, head, t, ct)
        onll, olse, _ = olce.forward(h.cuda(), wdq.cuda(), t.cuda(), dtype=torch.float64)
        odh = olce.backward(h.cuda(), wdq.cuda(), t.cuda(), olse, ct.cuda(), round_g_bf16=False, dtype=torch.float64)
        e_nll = float((nll - onll.cpu()).abs().max())
        r_dh = rel_l2(dh, odh.cpu())
        print(f"  scales {sdt}: nll max-abs {e_nll:.2e}, dH rel-L2 {r_dh:.2e}", flush=True)
        assert e_nll < 1e-5 and r_dh < 1e-5


ATT_SHAPES = [  # (b, hq, hkv, s, d): the reference's head x N cases plus head_dim 96 / 128 and B = 2
    (1, 4, 4, 64, 64), (1, 4, 4, 61, 64), (1, 4, 4, 257, 64), (1, 4, 2, 61, 64), (1, 4, 2, 257, 64),
    (1, 32, 8, 64, 128), (2, 4, 2, 130, 128), (1, 4, 1, 100, 96),
]


def _attn32(q, k, v, do, scale, *, causal=True, sid=None, sst=None):
    from mlx_train_perf.attention.api import kernel_backward, kernel_forward

    qd, kd, vd, dod = (x.cuda().contiguous() for x in (q, k, v, do))
    sd = None if sid is None else sid.cuda().int().contiguous()
    ss = None if sst is None else sst.cuda().int().contiguous()
    o, lse = kernel_forward(qd, kd, vd, scale=scale, seg_id=sd, seg_start=ss, causal=causal)
    dq, dk, dv = kernel_backward(qd, kd, vd, o, lse, dod, scale=scale, seg_id=sd, seg_start=ss, causal=causal)
    torch.cuda.synchronize()
    return [x.cpu().double() for x in (o, lse, dq, dk, dv)]


def _attn_check(got, q, k, v, do, scale, *, causal=True, sid=None, tag=""):
    oo, ol = oatt.attention_forward(q.cuda(), k.cuda(), v.cuda(), scale=scale, causal=causal,
                                    seg_id=None if sid is None else sid.cuda(), dtype=torch.float64)
    odq, odk, odv = oatt.attention_backward(q.cuda(), k.cuda(), v.cuda(), oo, ol, do.cuda(), scale=scale,
                                            causal=causal, seg_id=None if sid is None else sid.cuda(),
                                            dtype=torch.float64)
    o, lse, dq, dk, dv = got
    e = {name: float((a - b.cpu()).abs().max())
         for name, a, b in (("O", o, oo), ("L", lse, ol), ("dQ", dq, odq), ("dK", dk, odk), ("dV", dv, odv))}
    print(f"  {tag} " + ", ".join(f"{k_} {v_:.2e}" for k_, v_ in e.items()), flush=True)
    assert e["O"] < 2e-6 and e["L"] < 2e-6 and e["dQ"] < 5e-6 and e["dK"] < 2.5e-5 and e["dV"] < 2.5e-5, e


@pytest.mark.parametrize("shape", ATT_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
def test_attention_fp32_parity(shape, causal):
    b, hq, hkv, s, d = shape
    print(f"[attention fp32 {shape} causal={causal}]", flush=True)
    g = torch.Generator().manual_seed(41)
    q = torch.randn(b, hq, s, d, generator=g)
    k = torch.randn(b, hkv, s, d, generator=g)
    v = torch.randn(b, hkv, s, d, generator=g)
    do = torch.randn(b, hq, s, d, generator=g)
    scale = 1 / math.sqrt(d)
    _attn_check(_attn32(q, k, v, do, scale, causal=causal), q, k, v, do, scale, causal=causal, tag=str(shape))


@pytest.mark.parametrize("lengths", [[5, 7], [1, 60, 3, 200], [257], [40, 1, 1, 88]])
def test_attention_fp32_packed(lengths):
    """Packed rows (B = 2) against the block-diagonal oracle; one segment equals plain causal
    bitwise."""
    print(f"[attention fp32 packed {lengths}]", flush=True)
    s = sum(lengths)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 4, s, 64, generator=g)
    k = torch.randn(2, 2, s, 64, generator=g)
    v = torch.randn(2, 2, s, 64, generator=g)
    do = torch.randn(2, 4, s, 64, generator=g)
    sid, sst = oatt.segments_from_lengths(lengths)
    sid2, sst2 = sid[None].repeat(2, 1), sst[None].repeat(2, 1)
    got = _attn32(q, k, v, do, 0.125, sid=sid2, sst=sst2)
    _attn_check(got, q, k, v, do, 0.125, sid=sid2, tag="packed")
    if len(lengths) == 1:
        plain = _attn32(q, k, v, do, 0.125)
        assert all(torch.equal(a, b_) for a, b_ in zip(got, plain))


def test_flash_attention_fp32_public_api():
    """flash_attention resolves fp32 to the kernel (no refusal, no fallback) and its autograd matches
    the oracle at the fp32 bar."""
    from mlx_train_perf.attention import flash_attention
    from mlx_train_perf.attention.api import VJP_CALLS, resolve_attention_impl

    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 4, 96, 64, generator=g)
    k = torch.randn(1, 2, 96, 64, generator=g)
    v = torch.randn(1, 2, 96, 64, generator=g)
    do = torch.randn(1, 4, 96, 64, generator=g)
    qd, kd, vd = (x.cuda().requires_grad_(True) for x in (q, k, v))
    assert resolve_attention_impl(qd, kd, vd, impl="auto") == "kernel"
    before = VJP_CALLS.get("flash_attention_kernel_bwd", 0)
    o = flash_attention(qd, kd, vd, scale=0.125)
    o.backward(do.cuda())
    assert VJP_CALLS.get("flash_attention_kernel_bwd", 0) == before + 1
    assert o.dtype == torch.float32 and qd.grad.dtype == torch.float32
    got = [o.detach().cpu().double(), None, qd.grad.cpu().double(), kd.grad.cpu().double(), vd.grad.cpu().double()]
    oo, ol = oatt.attention_forward(q, k, v, scale=0.125, dtype=torch.float64)
    odq, odk, odv = oatt.attention_backward(q, k, v, oo, ol, do, scale=0.125, dtype=torch.float64)
    assert float((got[0] - oo).abs().max()) < 2e-6
    assert float((got[2] - odq).abs().max()) < 5e-6
    assert float((got[3] - odk).abs().max()) < 2.5e-5 and float((got[4] - odv).abs().max()) < 2.5e-5


# Seeded random shapes (fixed by the seed): ragged n, v and any hidden dim for the dense head
# (fp32 rows need no multiple of 8), 4-bit heads at multiples of 64, trainable heads, and attention
# with GQA ratios 1-4, causal and non-causal, and packed rows. Bars: nll 2e-5 max-abs (values up to
# ~9 at v = 6000), dH / dW / O / dQ / dK / dV 1e-5 relative-L2, L 1e-5 max-abs.
_R = _random.Random(3232)
RAND_LCE = []
for _ in range(8):
    _kind = _R.choice(["dense", "dense", "q4", "trainable"])
    _d = _R.choice([64, 128, 192, 256, 512]) if _kind == "q4" else _R.choice([1, 3, 17, 32, 64, 100, 200, 512])
    RAND_LCE.append((_kind, _R.randint(1, 700), _d, _R.randint(1, 6000)))
RAND_ATT = []
for _ in range(8):
    _hkv, _g = _R.choice([1, 2, 4]), _R.choice([1, 2, 3, 4])
    RAND_ATT.append((_R.randint(1, 2), _hkv * _g, _hkv, _R.randint(1, 400), _R.choice([64, 96, 128]),
                     _R.choice([True, False])))
RAND_PACKED = [[_R.randint(1, 150) for _ in range(_R.randint(1, 5))] for _ in range(4)]


@pytest.mark.parametrize(("kind", "n", "d", "v"), RAND_LCE)
def test_lce_fp32_random(kind, n, d, v):
    from mlx_train_perf import DenseHead, QuantizedHead, linear_cross_entropy

    print(f"[lce fp32 random {kind} n={n} d={d} v={v}]", flush=True)
    g = torch.Generator().manual_seed(n * 7 + d + v)
    h = torch.randn(n, d, generator=g)
    w = torch.randn(v, d, generator=g) * 0.05
    t = torch.randint(0, v, (n,), generator=g)
    t[torch.randperm(n, generator=g)[: n // 10]] = IGN
    valid = t != IGN
    ct = valid.double() / valid.sum().clamp(min=1)
    if kind == "q4":
        wq, sc, bi = oquant.quantize_affine(w, scale_dtype=torch.float32)
        w = oquant.dequantize_affine(wq, sc, bi, dtype=torch.float64).float()
        head = QuantizedHead(w_q=wq.cuda(), scales=sc.cuda(), biases=bi.cuda())
    wd = w.cuda().requires_grad_(kind == "trainable")
    if kind != "q4":
        head = DenseHead(weight=wd, trainable=kind == "trainable")
    hd = h.cuda().requires_grad_(True)
    nll = linear_cross_entropy(hd, head, t.cuda(), reduction="none")
    (nll * ct.cuda().float()).sum().backward()
    wc = w.double().cuda()
    onll, olse, _ = olce.forward(h.cuda(), wc, t.cuda(), dtype=torch.float64)
    odh = olce.backward(h.cuda(), wc, t.cuda(), olse, ct.cuda(), round_g_bf16=False, dtype=torch.float64)
    e_nll = float((nll.detach().cpu().double() - onll.cpu()).abs().max())
    r_dh = rel_l2(hd.grad.cpu(), odh.cpu()) if valid.any() else float(hd.grad.abs().max())
    print(f"  nll max-abs {e_nll:.2e}, dH rel-L2 {r_dh:.2e}", flush=True)
    assert e_nll < 2e-5 and r_dh < 1e-5
    assert (hd.grad[~valid.cuda()] == 0).all()
    if kind == "trainable" and valid.any():
        odw = olce.backward_dw(h.cuda(), wc, t.cuda(), olse, ct.cuda(), round_g_bf16=False, dtype=torch.float64)
        r_dw = rel_l2(wd.grad.cpu(), odw.cpu())
        print(f"  dW rel-L2 {r_dw:.2e}", flush=True)
        assert r_dw < 1e-5


def _attn_check_rel(got, q, k, v, do, scale, *, causal=True, sid=None, tag=""):
    oo, ol = oatt.attention_forward(q.cuda(), k.cuda(), v.cuda(), scale=scale, causal=causal,
                                    seg_id=None if sid is None else sid.cuda(), dtype=torch.float64)
    odq, odk, odv = oatt.attention_backward(q.cuda(), k.cuda(), v.cuda(), oo, ol, do.cuda(), scale=scale,
                                            causal=causal, seg_id=None if sid is None else sid.cuda(),
                                            dtype=torch.float64)
    o, lse, dq, dk, dv = got
    e = {name: rel_l2(a, b.cpu()) for name, a, b in (("O", o, oo), ("dQ", dq, odq), ("dK", dk, odk), ("dV", dv, odv))
         if float(b.abs().max()) > 1e-12}   # s = 1: dQ and dK are exactly 0
    e["L"] = float((lse - ol.cpu()).abs().max())
    print(f"  {tag} " + ", ".join(f"{k_} {v_:.2e}" for k_, v_ in e.items()), flush=True)
    assert all(x < 1e-5 for x in e.values()), e


@pytest.mark.parametrize(("b", "hq", "hkv", "s", "d", "causal"), RAND_ATT)
def test_attention_fp32_random(b, hq, hkv, s, d, causal):
    print(f"[attention fp32 random b={b} hq={hq} hkv={hkv} s={s} d={d} causal={causal}]", flush=True)
    g = torch.Generator().manual_seed(b * 1000 + s + d)
    q = torch.randn(b, hq, s, d, generator=g)
    k = torch.randn(b, hkv, s, d, generator=g)
    v = torch.randn(b, hkv, s, d, generator=g)
    do = torch.randn(b, hq, s, d, generator=g)
    scale = 1 / math.sqrt(d)
    _attn_check_rel(_attn32(q, k, v, do, scale, causal=causal), q, k, v, do, scale, causal=causal, tag="random")


@pytest.mark.parametrize("lengths", RAND_PACKED)
def test_attention_fp32_random_packed(lengths):
    print(f"[attention fp32 random packed {lengths}]", flush=True)
    s = sum(lengths)
    g = torch.Generator().manual_seed(s)
    q = torch.randn(1, 8, s, 128, generator=g)
    k = torch.randn(1, 2, s, 128, generator=g)
    v = torch.randn(1, 2, s, 128, generator=g)
    do = torch.randn(1, 8, s, 128, generator=g)
    sid, sst = oatt.segments_from_lengths(lengths)
    got = _attn32(q, k, v, do, 0.09, sid=sid[None], sst=sst[None])
    _attn_check_rel(got, q, k, v, do, 0.09, sid=sid[None], tag="packed")
