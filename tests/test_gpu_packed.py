"""GPU: packed (block-diagonal causal) attention masking, beyond the parity grid of
test_gpu_attention.py.

- No cross-segment leakage, bitwise: perturbing Q, K, V and dO inside one document leaves every
  other document's O, L, dQ, dK and dV bit-for-bit unchanged (reference
  tests/test_attention_segments.py:32-57 states the per-segment identity; here it is checked on the
  kernels, with boundaries off the 64-position tiles and documents sharing waves and tiles).
- Batches whose rows carry different layouts (per-row seg pointers, the dK/dV per-row search).
- The parity check discriminates: the kernels' output measured against the oracle with a planted
  mistake -- segments ignored, a boundary moved by one position, the diagonal dropped -- must
  exceed the parity bar on the rows the mistake touches (reference
  tests/test_attention_kernel_fwd.py:600-669, 854-; the mistake is planted in the oracle, on the CPU,
  never in a kernel).
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oatt
from tests._inputs import attn_inputs, rel_l2

pytestmark = pytest.mark.gpu


def _layout(rows: list[list[int]]):
    sids, ssts = zip(*(oatt.segments_from_lengths(r) for r in rows))
    return torch.stack(sids), torch.stack(ssts)


def _run(q, k, v, do, scale, sid, sst):
    from mlx_train_perf.attention.api import kernel_backward, kernel_forward

    qd, kd, vd, dod = (x.cuda().contiguous() for x in (q, k, v, do))
    sd, td = sid.cuda().contiguous(), sst.cuda().contiguous()
    o, lse = kernel_forward(qd, kd, vd, scale=scale, seg_id=sd, seg_start=td)
    dq, dk, dv = kernel_backward(qd, kd, vd, o, lse, dod, scale=scale, seg_id=sd, seg_start=td)
    torch.cuda.synchronize()
    return [x.cpu() for x in (o, lse, dq, dk, dv)]


LEAK_ROWS = [
    [37, 100, 1, 77, 130, 66],          # row 0: boundaries at 37, 137, 138, 215, 345 (none 64-aligned)
    [200, 5, 59, 3, 144],               # row 1: another layout (per-row segment pointers)
]


@pytest.mark.parametrize(("d", "hq", "hkv"), [(128, 8, 2), (64, 4, 2), (96, 4, 1)])
def test_no_cross_segment_leakage_bitwise(d, hq, hkv):
    b, s = 2, 411
    print(f"[packed leakage] d={d} hq={hq} hkv={hkv} rows={LEAK_ROWS}", flush=True)
    sid, sst = _layout(LEAK_ROWS)
    q, k, v, do = attn_inputs(b, hq, hkv, s, d, seed=31 + d)
    scale = 1.0 / math.sqrt(d)
    base = _run(q, k, v, do, scale, sid, sst)
    # perturb document 3 of row 0 (positions 138..214) in every input, with a large spread so the
    # forward's running maxima of those rows move
    a, e = 138, 215
    g = torch.Generator().manual_seed(7)
    q2, k2, v2, do2 = (x.clone() for x in (q, k, v, do))
    for x in (q2, k2, v2, do2):
        x[0, :, a:e] = (torch.randn(x[0, :, a:e].shape, generator=g) * 2.0).to(x.dtype)
    pert = _run(q2, k2, v2, do2, scale, sid, sst)
    inside = torch.zeros(b, s, dtype=torch.bool)
    inside[0, a:e] = True
    names = ("O", "L", "dQ", "dK", "dV")
    for name, x, y in zip(names, base, pert):
        # positions outside the perturbed document: bitwise identical (row 1 entirely)
        # (b, heads, s[, d]) -> (b, s, heads[, d]), then select positions
        xo, yo = x.transpose(1, 2)[~inside], y.transpose(1, 2)[~inside]
        assert torch.equal(xo, yo), f"{name} changed outside the perturbed document"
        xi = x.transpose(1, 2)[inside]
        yi = y.transpose(1, 2)[inside]
        assert not torch.equal(xi, yi), f"{name} did not change inside the perturbed document"
    # and both runs are right
    for run, (qq, kk, vv, dd) in ((base, (q, k, v, do)), (pert, (q2, k2, v2, do2))):
        oo, ol = oatt.attention_forward(qq, kk, vv, scale=scale, seg_id=sid, dtype=torch.float64)
        grads = oatt.attention_backward(qq, kk, vv, oo, ol, dd, scale=scale, seg_id=sid, dtype=torch.float64)
        assert rel_l2(run[0], oo) <= 1e-2 and float((run[1].double() - ol).abs().max()) <= 2e-3
        for got, want in zip(run[2:], grads):
            assert rel_l2(got, want) <= 1e-2


@pytest.mark.parametrize(("d", "hq", "hkv"), [(128, 8, 2), (64, 4, 2), (96, 6, 3)])
def test_batch_rows_with_different_layouts(d, hq, hkv):
    rows = [[120, 3, 200, 77], [1, 64, 64, 65, 206], [400]]
    b, s = len(rows), 400
    print(f"[packed b={b}] d={d} hq={hq} hkv={hkv} rows={rows}", flush=True)
    sid, sst = _layout(rows)
    q, k, v, do = attn_inputs(b, hq, hkv, s, d, seed=5 + d)
    scale = 1.0 / math.sqrt(d)
    o, lse, dq, dk, dv = _run(q, k, v, do, scale, sid, sst)
    oo, ol = oatt.attention_forward(q, k, v, scale=scale, seg_id=sid, dtype=torch.float64)
    gq, gk, gv = oatt.attention_backward(q, k, v, oo, ol, do, scale=scale, seg_id=sid, dtype=torch.float64)
    assert rel_l2(o, oo) <= 1e-2
    assert float((o.double() - oo).abs().max()) <= 1.2e-2 * max(1.0, float(oo.abs().max()))
    assert float((lse.double() - ol).abs().max()) <= 2e-3
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        assert rel_l2(got, want) <= 1e-2
    # each row alone (B=1) gives the same bits as inside the batch (when the dK/dV size table picks
    # the same split for B=1 as for B: the split sets the fp32 summation grouping of dK/dV)
    from mlx_train_perf.plan.launch import attn_dkv_splits

    assert attn_dkv_splits(b=1, hq=hq, hkv=hkv, s=s, dh=d) == attn_dkv_splits(b=b, hq=hq, hkv=hkv, s=s, dh=d)
    for r in range(b):
        one = _run(q[r:r + 1], k[r:r + 1], v[r:r + 1], do[r:r + 1], scale, sid[r:r + 1], sst[r:r + 1])
        for x, y in zip(one, (o, lse, dq, dk, dv)):
            assert torch.equal(x[0], y[r])


def _planted(q, k, v, scale, rule: str, lens: list[int]):
    """The oracle's forward with a mistake planted in its mask (CPU, fp64): "causal" ignores the
    segments, "moved" starts document 1 one position early, "nodiag" hides the diagonal key."""
    s = q.shape[2]
    if rule == "causal":
        return oatt.attention_forward(q, k, v, scale=scale, dtype=torch.float64)
    if rule == "moved":
        moved = [lens[0] - 1, lens[1] + 1] + lens[2:]
        sid, _ = oatt.segments_from_lengths(moved)
        return oatt.attention_forward(q, k, v, scale=scale, seg_id=sid[None], dtype=torch.float64)
    sid, _ = oatt.segments_from_lengths(lens)
    allowed = oatt.segment_allowed(sid[None]) & ~torch.eye(s, dtype=torch.bool)[None, None]
    hq = q.shape[1]
    kg = k.repeat_interleave(hq // k.shape[1], dim=1).double()
    vg = v.repeat_interleave(hq // v.shape[1], dim=1).double()
    sc = (q.double() @ kg.transpose(-1, -2).contiguous()) * scale
    sc = sc.masked_fill(~allowed, float("-inf"))
    lse = torch.logsumexp(sc, dim=-1)
    return torch.exp(sc - lse[..., None]) @ vg, lse


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("rule", ["causal", "moved", "nodiag"])
def test_parity_check_rejects_planted_mask_mistakes(rule, d):
    lens = [70, 90, 43]
    s = sum(lens)
    print(f"[packed must-fail] rule={rule} d={d} lens={lens}", flush=True)
    q, k, v, do = attn_inputs(1, 4, 2, s, d, seed=17)
    scale = 1.0 / math.sqrt(d)
    sid, sst = _layout([lens])
    o, lse, *_ = _run(q, k, v, do, scale, sid, sst)
    good_o, good_l = oatt.attention_forward(q, k, v, scale=scale, seg_id=sid, dtype=torch.float64)
    assert float((o.double() - good_o).abs().max()) <= 1.2e-2      # the true oracle passes
    bad_o, bad_l = _planted(q, k, v, scale, rule, lens)
    # rows the mistake touches (finite in the planted oracle): document 1 onward for "causal",
    # document 1 (and the moved row) for "moved", every row but each document's first for "nodiag"
    if rule == "nodiag":
        rows = torch.ones(s, dtype=torch.bool)
        rows[[0, lens[0], lens[0] + lens[1]]] = False
    else:
        rows = torch.zeros(s, dtype=torch.bool)
        rows[lens[0] - (1 if rule == "moved" else 0):lens[0] + lens[1]] = True
    d_o = float((o[:, :, rows].double() - bad_o[:, :, rows]).abs().max())
    d_l = float((lse[:, :, rows].double() - bad_l[:, :, rows]).abs().max())
    print(f"  vs planted oracle: O max-abs {d_o:.3e}, L max-abs {d_l:.3e}", flush=True)
    assert torch.isfinite(bad_o[:, :, rows]).all()
    assert d_o > 10 * 1.2e-2 or d_l > 10 * 2e-3
