"""The CPU oracle still reproduces the committed golden fixtures (regression pin of the checker)."""
from __future__ import annotations

import torch

from oracle import attention as oa
from oracle import lce as olce
from oracle import quant as oq
from tests._golden import load


def test_lce_dense_fixture():
    g = load("lce_dense_n64_d64_v1024.npz")
    nll, lse, tgt = olce.forward(g["hidden"], g["weight"], g["targets"])
    assert torch.allclose(nll, g["nll"], atol=1e-12) and torch.allclose(lse, g["lse"], atol=1e-12)
    assert torch.equal(tgt == 0, g["tgt"] == 0)
    dh = olce.backward(g["hidden"], g["weight"], g["targets"], lse, g["cotangent"], dtype=torch.float64)
    assert torch.allclose(dh, g["d_hidden"], atol=1e-12)


def test_lce_q4_fixture():
    g = load("lce_q4_n32_d128_v512.npz")
    wdq = oq.dequantize_affine(g["w_q"], g["scales"], g["biases"])
    nll, lse, _ = olce.forward(g["hidden"], wdq, g["targets"])
    assert torch.allclose(nll, g["nll"], atol=1e-12)
    dh = olce.backward(g["hidden"], wdq, g["targets"], lse, g["cotangent"], dtype=torch.float64)
    assert torch.allclose(dh, g["d_hidden"], atol=1e-12)


def test_attention_fixtures():
    for name in ("attn_causal_b1_hq4_hkv2_s61_d64.npz", "attn_packed_b1_hq4_hkv2_s61_d64.npz"):
        g = load(name)
        sid = g.get("seg_id")
        scale = float(g["scale"])
        o, lse = oa.attention_forward(g["q"], g["k"], g["v"], scale=scale, seg_id=sid, dtype=torch.float64)
        assert torch.allclose(o, g["o"], atol=1e-12) and torch.allclose(lse, g["lse"], atol=1e-12)
        grads = oa.attention_backward(g["q"], g["k"], g["v"], o, lse, g["d_o"], scale=scale, seg_id=sid,
                                      dtype=torch.float64)
        for got, key in zip(grads, ("dq", "dk", "dv")):
            assert torch.allclose(got, g[key], atol=1e-12)
