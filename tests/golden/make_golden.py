"""Generate the committed golden fixtures from the CPU oracle (run from the repository root):

    python tests/golden/make_golden.py

Each .npz holds the seeded inputs (bf16 as uint16 bit patterns, integer tensors as int32/int64) and
the oracle's fp64 outputs. The CPU lane checks the oracle still reproduces them; the GPU lane checks
the HIP kernels against them at the stated tolerances.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention as oa  # noqa: E402
from oracle import lce as olce  # noqa: E402
from oracle import quant as oq  # noqa: E402
from tests._inputs import attn_inputs, lce_inputs  # noqa: E402

OUT = Path(__file__).resolve().parent


def u16(x: torch.Tensor) -> np.ndarray:
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def lce_dense():
    h, w, t = lce_inputs(64, 64, 1024, seed=123, ignore_frac=0.1)
    ct = torch.rand(64, generator=torch.Generator().manual_seed(7)) + 0.5
    nll, lse, tgt = olce.forward(h, w, t)
    dh = olce.backward(h, w, t, lse, ct, round_g_bf16=True, dtype=torch.float64)
    np.savez_compressed(OUT / "lce_dense_n64_d64_v1024.npz", hidden=u16(h), weight=u16(w), targets=t.numpy(),
                        cotangent=ct.numpy(), nll=nll.numpy(), lse=lse.numpy(), tgt=tgt.numpy(), d_hidden=dh.numpy())


def lce_q4():
    h, w, t = lce_inputs(32, 128, 512, seed=321, ignore_frac=0.1, w_std=0.05)
    wq, sc, bi = oq.quantize_affine(w.float(), scale_dtype=torch.bfloat16)
    wdq = oq.dequantize_affine(wq, sc, bi)
    ct = torch.rand(32, generator=torch.Generator().manual_seed(8)) + 0.5
    nll, lse, tgt = olce.forward(h, wdq, t)
    dh = olce.backward(h, wdq, t, lse, ct, round_g_bf16=True, dtype=torch.float64)
    np.savez_compressed(OUT / "lce_q4_n32_d128_v512.npz", hidden=u16(h), w_q=wq.numpy(), scales=u16(sc),
                        biases=u16(bi), targets=t.numpy(), cotangent=ct.numpy(), nll=nll.numpy(), lse=lse.numpy(),
                        tgt=tgt.numpy(), d_hidden=dh.numpy())


def attention(name, lengths=None):
    b, hq, hkv, s, d = 1, 4, 2, 61, 64
    q, k, v, do = attn_inputs(b, hq, hkv, s, d, seed=61)
    scale = 0.125
    sid = sst = None
    if lengths:
        sid, sst = oa.segments_from_lengths(lengths)
        sid, sst = sid[None], sst[None]
    o, lse = oa.attention_forward(q, k, v, scale=scale, seg_id=sid, dtype=torch.float64)
    dq, dk, dv = oa.attention_backward(q, k, v, o, lse, do, scale=scale, seg_id=sid, dtype=torch.float64)
    extra = {} if sid is None else {"seg_id": sid.numpy(), "seg_start": sst.numpy()}
    np.savez_compressed(OUT / name, q=u16(q), k=u16(k), v=u16(v), d_o=u16(do), scale=np.float64(scale), o=o.numpy(),
                        lse=lse.numpy(), dq=dq.numpy(), dk=dk.numpy(), dv=dv.numpy(), **extra)


if __name__ == "__main__":
    torch.manual_seed(0)
    lce_dense()
    lce_q4()
    attention("attn_causal_b1_hq4_hkv2_s61_d64.npz")
    attention("attn_packed_b1_hq4_hkv2_s61_d64.npz", lengths=[20, 1, 40])
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))
