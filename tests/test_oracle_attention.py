"""Pins for the attention oracle (oracle/attention.py) on the CPU.

Mirrors the reference's oracle tests: row-0 closed form (tests/test_attention_kernel_fwd.py:522-544),
the constant-V GQA discriminator (tests/test_attention_reference.py:111-136), L against an
independently built logsumexp (:56-80), the finite-difference gradient anchor (:139-202), the 4x4
segment_allowed KAT (tests/test_attention_segments.py:68-87) and per-segment composition of the
packed forward and backward (:32-57, 90-131).
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oa


def _qkv(b=1, hq=4, hkv=2, n=9, d=8, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(s, generator=g, dtype=dtype) for s in ((b, hq, n, d), (b, hkv, n, d), (b, hkv, n, d)))


def test_row0_attends_only_to_itself():
    q, k, v = _qkv()
    o, lse = oa.attention_forward(q, k, v, scale=0.3, dtype=torch.float64)
    for h in range(4):
        kv = oa.kv_head_for(h, 2)
        assert torch.allclose(o[0, h, 0], v[0, kv, 0])
        assert abs(lse[0, h, 0].item() - 0.3 * float(q[0, h, 0] @ k[0, kv, 0])) < 1e-12


def test_constant_v_gqa_discriminator():
    # V constant per kv head: every output row of head h must equal kv_head_for(h)'s constant,
    # which distinguishes contiguous grouping from interleaved grouping.
    q, k, _ = _qkv(hq=8, hkv=2)
    v = torch.empty(1, 2, 9, 8, dtype=torch.float64)
    v[0, 0], v[0, 1] = 1.0, 2.0
    o, _ = oa.attention_forward(q, k, v, scale=0.5, dtype=torch.float64)
    for h in range(8):
        assert torch.allclose(o[0, h], torch.full_like(o[0, h], 1.0 + (h // 4)))


def test_lse_matches_independent_logsumexp():
    q, k, v = _qkv(hq=2, hkv=1, n=6)
    _, lse = oa.attention_forward(q, k, v, scale=0.7, dtype=torch.float64)
    for h in range(2):
        for i in range(6):
            s = [0.7 * float(q[0, h, i] @ k[0, 0, j]) for j in range(i + 1)]
            m = max(s)
            assert abs(lse[0, h, i].item() - (m + math.log(sum(math.exp(x - m) for x in s)))) < 1e-12


def test_backward_matches_autograd_and_finite_differences():
    q, k, v = _qkv(hq=4, hkv=2, n=7, d=4, seed=3)
    do = torch.randn(1, 4, 7, 4, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    o, lse = oa.attention_forward(q, k, v, scale=0.5, dtype=torch.float64)
    dq, dk, dv = oa.attention_backward(q, k, v, o, lse, do, scale=0.5, dtype=torch.float64)
    qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
    oo, _ = oa.attention_forward(qq, kk, vv, scale=0.5, dtype=torch.float64)
    (oo * do).sum().backward()
    for got, want in ((dq, qq.grad), (dk, kk.grad), (dv, vv.grad)):
        assert torch.allclose(got, want, atol=1e-12)
    eps = 1e-6
    for idx in [(0, 1, 3, 2), (0, 0, 6, 0)]:
        kp, km = k.clone(), k.clone()
        kp[idx] += eps
        km[idx] -= eps
        fp = (oa.attention_forward(q, kp, v, scale=0.5, dtype=torch.float64)[0] * do).sum()
        fm = (oa.attention_forward(q, km, v, scale=0.5, dtype=torch.float64)[0] * do).sum()
        assert abs(((fp - fm) / (2 * eps)).item() - dk[idx].item()) < 1e-7


def test_planted_mistake_in_backward_fails():
    """Dropping the D term from dS must break the autograd agreement."""
    q, k, v = _qkv(hq=2, hkv=1, n=6, d=4, seed=5)
    do = torch.randn(1, 2, 6, 4, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    o, lse = oa.attention_forward(q, k, v, scale=0.5, dtype=torch.float64)
    dq, _, _ = oa.attention_backward(q, k, v, o, lse, do, scale=0.5, dtype=torch.float64)
    s = oa._scores(q, k, scale=0.5, causal=True, seg_id=None, dtype=torch.float64)
    p = torch.exp(s - lse[..., None])
    kg = oa._gather_kv(k, 2)
    dp = do @ oa._gather_kv(v, 2).transpose(-1, -2)
    bad = 0.5 * ((p * dp) @ kg)  # missing "- D"
    assert not torch.allclose(bad, dq, atol=1e-6)


def test_segment_allowed_kat():
    seg = torch.tensor([[0, 0, 1, 1]])
    want = torch.tensor([[1, 0, 0, 0], [1, 1, 0, 0], [0, 0, 1, 0], [0, 0, 1, 1]], dtype=torch.bool)
    assert torch.equal(oa.segment_allowed(seg)[0, 0], want)


@pytest.mark.parametrize("lengths", [[3, 5], [1, 4, 2], [6]])
def test_packed_equals_per_segment_composition(lengths):
    n = sum(lengths)
    q, k, v = _qkv(hq=2, hkv=1, n=n, d=4, seed=len(lengths))
    do = torch.randn(1, 2, n, 4, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    sid, _ = oa.segments_from_lengths(lengths)
    o, lse = oa.attention_forward(q, k, v, scale=0.5, seg_id=sid[None], dtype=torch.float64)
    grads = oa.attention_backward(q, k, v, o, lse, do, scale=0.5, seg_id=sid[None], dtype=torch.float64)
    pos = 0
    for ln in lengths:
        sl = slice(pos, pos + ln)
        oi, li = oa.attention_forward(q[:, :, sl], k[:, :, sl], v[:, :, sl], scale=0.5, dtype=torch.float64)
        gi = oa.attention_backward(q[:, :, sl], k[:, :, sl], v[:, :, sl], oi, li, do[:, :, sl], scale=0.5,
                                   dtype=torch.float64)
        assert torch.allclose(o[:, :, sl], oi, atol=1e-12) and torch.allclose(lse[:, :, sl], li, atol=1e-12)
        for gp, gs in zip(grads, gi):
            assert torch.allclose(gp[:, :, sl], gs, atol=1e-12)
        pos += ln


def test_single_segment_is_causal():
    q, k, v = _qkv(n=8)
    sid, _ = oa.segments_from_lengths([8])
    a = oa.attention_forward(q, k, v, scale=0.4, seg_id=sid[None], dtype=torch.float64)
    b = oa.attention_forward(q, k, v, scale=0.4, dtype=torch.float64)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_packed_layout_generator():
    lens = oa.packed_layout(16384, 64, 2048, seed=0)
    assert sum(lens) == 16384
    # every document drawn in [64, 2048]; only the last is truncated to fill the row exactly
    assert all(64 <= n <= 2048 for n in lens[:-1]) and 1 <= lens[-1] <= 2048
    assert sum(lens[:-1]) < 16384
    # the seed-0 layout: 13 documents and 12,388,368 visible pairs per head (the Python
    # random.Random(0) figures quoted for the packed workload, 134.2M when fully causal)
    assert len(lens) == 13
    assert sum(n * (n + 1) // 2 for n in lens) == 12_388_368
    sid, sst = oa.segments_from_lengths(lens)
    assert sid[0] == 0 and (sid[1:] >= sid[:-1]).all() and (sst[1:] >= sst[:-1]).all()
    assert (sst <= torch.arange(16384)).all()
    # gapless ids (steps of 0 or 1) and seg_start = the first position holding the same id
    assert set((sid[1:] - sid[:-1]).tolist()) <= {0, 1}
    first = {}
    for i, s_ in enumerate(sid.tolist()):
        first.setdefault(s_, i)
    assert sst.tolist() == [first[s_] for s_ in sid.tolist()]
    # a different seed gives a different layout (the seed is used)
    assert oa.packed_layout(16384, 64, 2048, seed=1) != lens
