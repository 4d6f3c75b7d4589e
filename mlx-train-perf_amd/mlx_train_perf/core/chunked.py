"""`impl="chunked"`: linear cross-entropy in plain torch ops over vocab slabs.

No more than one (N, slab) block of logits exists at a time. The head is read through `_Slabs`,
which hands out weight blocks in vocab order: a dense head is sliced, a 4-bit head has only the
requested block dequantized. One autograd Function does the rest:

- forward: a streaming log-sum-exp over the slabs (a running row maximum and a sum of exponentials
  rescaled whenever the maximum rises, so each slab is exponentiated once), the target logit picked
  from the slab that holds it, and the resulting `lse` saved as the only residual besides the inputs;
- backward: each slab again, p = exp(z - lse) with the target's indicator subtracted, scaled by the
  cotangent and rounded to the head dtype, then dL/dH += g @ W_slab in an fp32 accumulator and, for a
  trainable dense head, dL/dW[slab] = g^T @ H written in place.

The arithmetic is the reference's chunked path (src/mlx_train_perf/core/chunked.py:35-90: fp32
logits, g cast to the weight dtype before its product, fp32 dH accumulation, one cast at the end,
dW = g^T h per chunk). The one structural difference: the reference's custom vjp recomputes lse
(chunked.py:118-121); here it is saved by the forward, as the kernel path does. An explicit opt-in
only: it runs on whatever device holds the tensors and is never chosen by `impl="auto"`.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from mlx_train_perf.core.quant import dequantize


class QuantSpec(NamedTuple):
    """A frozen 4-bit affine head in the form this path reads it: packed words (V, D/8), per-group
    scale and bias (V, D/group_size), group size and bit width (reference core/chunked.py:16-22)."""
    w_q: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    group_size: int
    bits: int


# Test seam: each custom backward bumps its key ("dense" / "quantized") when it runs, so a test can
# tell the hand-written backward from an autograd trace through the forward ops.
VJP_CALLS: dict[str, int] = {}


class _Slabs:
    """Vocab slabs [v0, v1) of a head of `v` rows, `slab` rows each (the last one shorter)."""

    def __init__(self, *, v: int, slab: int, quant: QuantSpec | None, dtype: torch.dtype):
        if slab < 1:
            raise ValueError(f"chunk_size must be >= 1 (got {slab})")
        self.v, self.slab, self.quant, self.dtype = v, slab, quant, dtype

    def bounds(self):
        return ((v0, min(v0 + self.slab, self.v)) for v0 in range(0, self.v, self.slab))

    def weight(self, v0: int, v1: int, dense: torch.Tensor | None) -> torch.Tensor:
        if self.quant is None:
            return dense[v0:v1]
        q = self.quant
        return dequantize(q.w_q[v0:v1], q.scales[v0:v1], q.biases[v0:v1], group_size=q.group_size, bits=q.bits,
                          dtype=self.dtype)


def _slab_logits(hidden: torch.Tensor, w_slab: torch.Tensor) -> torch.Tensor:
    return (hidden @ w_slab.T).to(torch.float32)


def _target_column(targets: torch.Tensor, v0: int, v1: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(in-slab flag, clamped column index) of each row's target for slab [v0, v1)."""
    inside = (targets >= v0) & (targets < v1)
    return inside, (targets - v0).clamp(0, v1 - v0 - 1)


class _ChunkedLCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, dense_w, targets, slabs):
        n = hidden.shape[0]
        dev = hidden.device
        row_max = torch.full((n,), float("-inf"), dtype=torch.float32, device=dev)
        row_sum = torch.zeros((n,), dtype=torch.float32, device=dev)
        tgt = torch.zeros((n,), dtype=torch.float32, device=dev)
        for v0, v1 in slabs.bounds():
            z = _slab_logits(hidden, slabs.weight(v0, v1, dense_w))
            new_max = torch.maximum(row_max, z.amax(dim=-1))
            row_sum = row_sum * torch.exp(row_max - new_max) + torch.exp(z - new_max[:, None]).sum(dim=-1)
            row_max = new_max
            inside, col = _target_column(targets, v0, v1)
            tgt = torch.where(inside, z.gather(1, col[:, None]).squeeze(1), tgt)
        lse = row_max + torch.log(row_sum)
        ctx.save_for_backward(hidden, dense_w, targets, lse)
        ctx.slabs = slabs
        return lse - tgt

    @staticmethod
    def backward(ctx, grad_nll):
        hidden, dense_w, targets, lse = ctx.saved_tensors
        slabs: _Slabs = ctx.slabs
        VJP_CALLS["quantized" if slabs.quant is not None else "dense"] = \
            VJP_CALLS.get("quantized" if slabs.quant is not None else "dense", 0) + 1
        want_dw = dense_w is not None and ctx.needs_input_grad[1]
        ct = grad_nll.to(torch.float32)[:, None]
        dh32 = torch.zeros(hidden.shape, dtype=torch.float32, device=hidden.device)
        dw = torch.empty_like(dense_w) if want_dw else None
        for v0, v1 in slabs.bounds():
            w_slab = slabs.weight(v0, v1, dense_w)
            g = torch.exp(_slab_logits(hidden, w_slab) - lse[:, None])
            inside, col = _target_column(targets, v0, v1)
            g.scatter_add_(1, col[:, None], -inside.to(g.dtype)[:, None])
            g = (g * ct).to(w_slab.dtype)
            dh32 += (g @ w_slab).to(torch.float32)
            if want_dw:
                dw[v0:v1] = g.T @ hidden
        return dh32.to(hidden.dtype), dw, None, None


def chunked_nll(hidden: torch.Tensor, targets: torch.Tensor, *, chunk_size: int,
                weight: torch.Tensor | None = None, quant: QuantSpec | None = None) -> torch.Tensor:
    """Per-token NLL (N,) fp32 of `hidden` (N, D) against a dense `weight` (V, D) -- differentiable in
    both, so a trainable head gets its gradient -- or a frozen 4-bit `quant` head (dL/dH only).
    `targets` must lie in [0, V)."""
    if (weight is None) == (quant is None):
        raise ValueError("pass exactly one of weight= and quant=")
    v = weight.shape[0] if quant is None else quant.w_q.shape[0]
    slabs = _Slabs(v=v, slab=chunk_size, quant=quant, dtype=hidden.dtype)
    return _ChunkedLCE.apply(hidden, weight, targets.long(), slabs)
