"""GPU parity at the reference's published flagship workloads (C2-C5 below), through the C-ABI,
against the oracle in fp64.

The oracle (oracle/lce.py, oracle/attention.py) is device-agnostic torch; here it runs in fp64 on the
GPU so the full shapes finish in seconds:

- C2  LCE N=8192, D=4096, V=151936, bf16 head, H RMS-normalized, 5% ignore_index: per-token nll within
      2e-3 relative, lse likewise, the masked-mean loss within 2e-3 relative, dL/dH within 1e-2
      relative-L2, ignored rows exactly 0.
- C3  the same with the 4-bit affine (gs 64) head, against the fp32-dequantized head (the reference's
      fp32-head convention, tests/test_kernel_quant_parity.py:74-97): nll within 2e-3 relative and
      8e-3 absolute (the reference's bf16-dequant pin), dL/dH within 1e-2 relative-L2, through both
      backward paths (cached dequantized transposed head, and in-register dequant).
- Shapes past the flagship whose launches run several resident rounds of XCD rectangles (forward
  and gradient tiles at n=16384, v=65536; the dH product at n=16384, d=2048): same bars.
- C4  GQA causal attention B=1, Hq=32, Hkv=8, S=8192, head_dim 128: O, dQ, dK, dV within 1e-2
      relative-L2, O within 1.2e-2 x max(1, |O|max) max-abs (the reference's bf16 forward pin), L
      within 2e-3; the
      oracle runs one kv-head group (4 query heads) at a time.
- C5  packed attention, total 16384, document lengths uniform in [64, 2048] from seed 0 (13
      documents): same bars; the oracle is the per-document causal composition, which the CPU lane
      pins equal to the block-diagonal oracle (tests/test_oracle_attention.py).
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oatt
from oracle import lce as olce
from oracle import quant as oquant

pytestmark = pytest.mark.gpu

N, D, V = 8192, 4096, 151936
IGN = -100


class _RelL2:
    """Accumulates ||a - b||^2 and ||b||^2 over slices, for a relative-L2 of the whole tensor."""

    def __init__(self):
        self.num = 0.0
        self.den = 0.0

    def add(self, got: torch.Tensor, want: torch.Tensor) -> None:
        d = got.double() - want.double()
        self.num += float((d * d).sum())
        self.den += float((want.double() ** 2).sum())

    def value(self) -> float:
        return math.sqrt(self.num / max(self.den, 1e-300))


def _rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    r = _RelL2()
    r.add(a, b)
    return r.value()


def _c2_inputs(seed: int = 0):
    """Config 2 (N=8192, D=4096, V=151936): H ~ N(0,1) RMS-normalized, W ~ N(0, 0.02^2), targets uniform in [0, V) with
    round(0.05 N) = 410 rows (a seeded permutation) set to ignore_index; generated on the GPU."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    h = torch.randn(N, D, generator=g, device="cuda")
    h = (h / torch.sqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    w = (torch.randn(V, D, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g, device="cuda")
    t[torch.randperm(N, generator=g, device="cuda")[: round(0.05 * N)]] = IGN
    return h, w, t


def _check_lce(nll, lse, dh, onll, olse, odh, t, *, nll_abs=None):
    ign = t == IGN
    assert int(ign.sum()) == 410
    assert torch.isfinite(lse).all() and torch.isfinite(dh.float()).all()
    err = (nll.double() - onll).abs()
    assert (err <= 2e-3 * onll.abs() + 1e-4).all(), f"nll: worst {float(err.max()):.3e}"
    if nll_abs is not None:
        assert float(err.max()) <= nll_abs
    assert float((lse.double() - olse).abs().max()) <= 2e-3 * float(olse.abs().max())
    assert (nll[ign] == 0).all() and (dh[ign] == 0).all()
    valid = ~ign
    loss, oloss = nll[valid].double().mean(), olce.reduce_mean(onll, t)
    assert abs(float(loss - oloss)) <= 2e-3 * abs(float(oloss))
    r = _rel_l2(dh, odh)
    print(f"  nll max-abs {float(err.max()):.3e}, dH rel-L2 {r:.3e}", flush=True)
    assert r <= 1e-2


def _kernel_lce(h, head, t):
    from mlx_train_perf.core.loss import kernel_forward_parts

    valid = t != IGN
    ct = (valid.float() / valid.sum()).contiguous()   # cotangent of the masked mean
    hd = h.detach().clone().requires_grad_(True)
    nll, lse, _ = kernel_forward_parts(hd, head, t, ignore_index=IGN)
    nll.backward(ct)
    torch.cuda.synchronize()
    return nll.detach(), lse, hd.grad, ct


def test_c2_flagship_lce_dense():
    from mlx_train_perf import DenseHead, linear_cross_entropy

    print(f"[C2] lce dense N={N} D={D} V={V}", flush=True)
    h, w, t = _c2_inputs()
    head = DenseHead(weight=w, trainable=False)
    nll, lse, dh, ct = _kernel_lce(h, head, t)
    onll, olse, _ = olce.forward(h, w, t, ignore_index=IGN, dtype=torch.float64)
    odh = olce.backward(h, w, t, olse, ct, ignore_index=IGN, round_g_bf16=True, dtype=torch.float64)
    _check_lce(nll, lse, dh, onll, olse, odh, t)
    # the public entry point at the same shape: reduction="mean" and its gradient
    hd = h.detach().clone().requires_grad_(True)
    loss = linear_cross_entropy(hd, head, t, reduction="mean")
    loss.backward()
    oloss = olce.reduce_mean(onll, t)
    assert abs(loss.item() - oloss.item()) <= 2e-3 * abs(oloss.item())
    assert _rel_l2(hd.grad, odh) <= 1e-2


def test_c3_flagship_lce_q4(monkeypatch):
    from mlx_train_perf import QuantizedHead
    from mlx_train_perf.core import loss as L

    print(f"[C3] lce 4-bit N={N} D={D} V={V}", flush=True)
    h, w, t = _c2_inputs()
    wq, sc, bi = oquant.quantize_affine(w.float(), group_size=64, scale_dtype=torch.bfloat16)
    del w
    wdq = oquant.dequantize_affine(wq, sc, bi, group_size=64, dtype=torch.float32)
    head = QuantizedHead(w_q=wq, scales=sc, biases=bi)
    # the default: the forward over the whole head dequantized into its workspace, the backward
    # staging each vocab chunk's dequantized rows and the chunk transposed in its workspace
    monkeypatch.delenv("MTP_LCE_TRANSPOSED_HEAD", raising=False)
    monkeypatch.delenv("MTP_LCE_STAGE_HEAD", raising=False)
    L.clear_transposed_head_cache()
    nll, lse, dh, ct = _kernel_lce(h, head, t)
    assert L.transposed_head_cache_bytes() == 0
    onll, olse, _ = olce.forward(h, wdq, t, ignore_index=IGN, dtype=torch.float64)
    odh = olce.backward(h, wdq, t, olse, ct, ignore_index=IGN, round_g_bf16=True, dtype=torch.float64)
    _check_lce(nll, lse, dh, onll, olse, odh, t, nll_abs=8e-3)
    # the other two backwards: the whole head kept as a cached transposed copy, and neither copy nor
    # staging (the packed words dequantized in registers, in the forward too: its nll and lse are
    # the staged forward's bit for bit)
    for copy, stage in (("1", "1"), ("0", "0")):
        print(f"[C3] backward with MTP_LCE_TRANSPOSED_HEAD={copy} MTP_LCE_STAGE_HEAD={stage}", flush=True)
        monkeypatch.setenv("MTP_LCE_TRANSPOSED_HEAD", copy)
        monkeypatch.setenv("MTP_LCE_STAGE_HEAD", stage)
        L.clear_transposed_head_cache()
        nll2, lse2, dh2, _ = _kernel_lce(h, head, t)
        assert torch.equal(nll2, nll) and torch.equal(lse2, lse)
        assert (dh2[t == IGN] == 0).all()
        r = _rel_l2(dh2, odh)
        print(f"  dH rel-L2 {r:.3e}", flush=True)
        assert r <= 1e-2


@pytest.mark.parametrize(("n", "d", "v"), [(16384, 64, 65536), (16384, 2048, 4096)])
def test_lce_multi_round_xcd_rectangles(n, d, v):
    """Grids of several resident rounds of 256 workgroups in XCD rectangles: at n=16384, v=65536 the
    forward takes 8 splits of 64 row tiles (2 rounds) and so do the gradient tiles of the two-chunk
    backward (whose dH products split their vocab contraction); at d=2048, v=4096 the one-chunk dH
    product has 64 x 8 output tiles (2 rounds)."""
    from mlx_train_perf.core.loss import DenseHead
    from mlx_train_perf.plan import launch as plan

    print(f"[lce rounds] N={n} D={d} V={v}", flush=True)
    rt = n // 256
    if v == 65536:
        assert plan.lce_fwd_splits(n, v) == 8 and rt * 8 == 2 * 256
        chunk = plan.lce_bwd_chunk(n, d, v, plan.DEFAULT_LCE_BWD_BUDGET)
        assert -(-v // chunk) == 2 and plan.lce_nsplit(n, chunk, 1) == 8
        assert plan.lce_dh_ksplit(n, d, chunk // 256) > 1
    else:
        assert plan.lce_bwd_row_block(n, d, v, plan.DEFAULT_LCE_BWD_BUDGET) == n and rt * (d // 256) == 2 * 256
    g = torch.Generator(device="cuda").manual_seed(n + d + v)
    h = torch.randn(n, d, generator=g, device="cuda")
    h = (h / torch.sqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    w = (torch.randn(v, d, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device="cuda")
    t[torch.randperm(n, generator=g, device="cuda")[: n // 20]] = IGN
    nll, lse, dh, ct = _kernel_lce(h, DenseHead(weight=w, trainable=False), t)
    onll, olse, _ = olce.forward(h, w, t, ignore_index=IGN, dtype=torch.float64)
    odh = olce.backward(h, w, t, olse, ct, ignore_index=IGN, round_g_bf16=True, dtype=torch.float64)
    err = (nll.double() - onll).abs()
    assert (err <= 2e-3 * onll.abs() + 1e-4).all(), f"nll: worst {float(err.max()):.3e}"
    assert float((lse.double() - olse).abs().max()) <= 2e-3 * float(olse.abs().max())
    ign = t == IGN
    assert (nll[ign] == 0).all() and (dh[ign] == 0).all()
    r = _rel_l2(dh, odh)
    print(f"  nll max-abs {float(err.max()):.3e}, dH rel-L2 {r:.3e}", flush=True)
    assert r <= 1e-2


def _attn_gpu_inputs(b, hq, hkv, s, d, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    mk = lambda h: torch.randn(b, h, s, d, generator=g, device="cuda").to(torch.bfloat16)  # noqa: E731
    return mk(hq), mk(hkv), mk(hkv), mk(hq)


def _kernel_attn(q, k, v, do, scale, sid=None, sst=None):
    from mlx_train_perf.attention.api import kernel_backward, kernel_forward

    o, lse = kernel_forward(q, k, v, scale=scale, seg_id=sid, seg_start=sst)
    dq, dk, dv = kernel_backward(q, k, v, o, lse, do, scale=scale, seg_id=sid, seg_start=sst)
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


def _assert_attn(stats, o_maxabs, o_peak, l_maxabs):
    """rel-L2 per tensor; O max-abs against the reference's 1.2e-2 bf16 pin scaled by max(1, |O|max)
    (short documents average few V rows, so |O| reaches ~3, where bf16 rounding of the output alone
    is ~1.2e-2), as in test_gpu_attention.py; L within 2e-3."""
    for name, r in stats.items():
        print(f"  {name} rel-L2 {r.value():.3e}", flush=True)
        assert r.value() <= 1e-2, name
    print(f"  O max-abs {o_maxabs:.3e} (|O| max {o_peak:.2f}), L max-abs {l_maxabs:.3e}", flush=True)
    assert o_maxabs <= 1.2e-2 * max(1.0, o_peak)
    assert l_maxabs <= 2e-3


def test_c4_flagship_causal_attention():
    b, hq, hkv, s, d = 1, 32, 8, 8192, 128
    print(f"[C4] attention causal b={b} hq={hq} hkv={hkv} s={s} d={d}", flush=True)
    scale = 1.0 / math.sqrt(d)
    q, k, v, do = _attn_gpu_inputs(b, hq, hkv, s, d, seed=0)
    o, lse, dq, dk, dv = _kernel_attn(q, k, v, do, scale)
    grp = hq // hkv
    stats = {n: _RelL2() for n in ("O", "dQ", "dK", "dV")}
    o_max = l_max = o_peak = 0.0
    for kvh in range(hkv):   # one kv-head group at a time: 4 x 8192^2 fp64 scores
        hs = slice(kvh * grp, (kvh + 1) * grp)
        ks = slice(kvh, kvh + 1)
        oo, ol = oatt.attention_forward(q[:, hs], k[:, ks], v[:, ks], scale=scale, dtype=torch.float64)
        gq, gk, gv = oatt.attention_backward(q[:, hs], k[:, ks], v[:, ks], oo, ol, do[:, hs], scale=scale,
                                             dtype=torch.float64)
        stats["O"].add(o[:, hs], oo)
        stats["dQ"].add(dq[:, hs], gq)
        stats["dK"].add(dk[:, ks], gk)
        stats["dV"].add(dv[:, ks], gv)
        o_max = max(o_max, float((o[:, hs].double() - oo).abs().max()))
        o_peak = max(o_peak, float(oo.abs().max()))
        l_max = max(l_max, float((lse[:, hs].double() - ol).abs().max()))
        del oo, ol, gq, gk, gv
    _assert_attn(stats, o_max, o_peak, l_max)


def test_c5_flagship_packed_attention():
    b, hq, hkv, s, d = 1, 32, 8, 16384, 128
    lens = oatt.packed_layout(s, 64, 2048, seed=0)
    print(f"[C5] attention packed s={s} segments={len(lens)} hq={hq} hkv={hkv} d={d}", flush=True)
    assert sum(lens) == s and len(lens) == 13
    scale = 1.0 / math.sqrt(d)
    q, k, v, do = _attn_gpu_inputs(b, hq, hkv, s, d, seed=1)
    sid, sst = (x[None].cuda() for x in oatt.segments_from_lengths(lens))
    o, lse, dq, dk, dv = _kernel_attn(q, k, v, do, scale, sid, sst)
    stats = {n: _RelL2() for n in ("O", "dQ", "dK", "dV")}
    o_max = l_max = o_peak = 0.0
    a = 0
    for n in lens:   # per-document causal oracle: each document sees only itself
        ps = slice(a, a + n)
        oo, ol = oatt.attention_forward(q[:, :, ps], k[:, :, ps], v[:, :, ps], scale=scale, dtype=torch.float64)
        gq, gk, gv = oatt.attention_backward(q[:, :, ps], k[:, :, ps], v[:, :, ps], oo, ol, do[:, :, ps],
                                             scale=scale, dtype=torch.float64)
        stats["O"].add(o[:, :, ps], oo)
        stats["dQ"].add(dq[:, :, ps], gq)
        stats["dK"].add(dk[:, :, ps], gk)
        stats["dV"].add(dv[:, :, ps], gv)
        o_max = max(o_max, float((o[:, :, ps].double() - oo).abs().max()))
        o_peak = max(o_peak, float(oo.abs().max()))
        l_max = max(l_max, float((lse[:, :, ps].double() - ol).abs().max()))
        a += n
    _assert_attn(stats, o_max, o_peak, l_max)


@pytest.mark.parametrize(("s", "d"), [(2048, 128), (4096, 128), (2048, 64), (4096, 96)])
def test_causal_attention_split_dkv_sizes(s, d):
    """The sizes where the dK/dV pass splits its key blocks (4 splits at 2048, 2 at 4096 for B=1,
    Hq=32, Hkv=8, any head_dim): fp32 partials summed by the reduce kernel, same bars as C4."""
    from mlx_train_perf.plan.launch import attn_dkv_splits

    b, hq, hkv = 1, 32, 8
    ns = attn_dkv_splits(b=b, hq=hq, hkv=hkv, s=s)
    print(f"[attn causal split dK/dV] s={s} d={d} splits={ns}", flush=True)
    assert ns == {2048: 4, 4096: 2}[s]
    scale = 1.0 / math.sqrt(d)
    q, k, v, do = _attn_gpu_inputs(b, hq, hkv, s, d, seed=s + d)
    o, lse, dq, dk, dv = _kernel_attn(q, k, v, do, scale)
    grp = hq // hkv
    stats = {n: _RelL2() for n in ("O", "dQ", "dK", "dV")}
    o_max = l_max = o_peak = 0.0
    for kvh in range(hkv):
        hs, ks = slice(kvh * grp, (kvh + 1) * grp), slice(kvh, kvh + 1)
        oo, ol = oatt.attention_forward(q[:, hs], k[:, ks], v[:, ks], scale=scale, dtype=torch.float64)
        gq, gk, gv = oatt.attention_backward(q[:, hs], k[:, ks], v[:, ks], oo, ol, do[:, hs], scale=scale,
                                             dtype=torch.float64)
        stats["O"].add(o[:, hs], oo)
        stats["dQ"].add(dq[:, hs], gq)
        stats["dK"].add(dk[:, ks], gk)
        stats["dV"].add(dv[:, ks], gv)
        o_max = max(o_max, float((o[:, hs].double() - oo).abs().max()))
        o_peak = max(o_peak, float(oo.abs().max()))
        l_max = max(l_max, float((lse[:, hs].double() - ol).abs().max()))
    _assert_attn(stats, o_max, o_peak, l_max)
