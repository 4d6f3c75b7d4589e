"""Chunked linear-CE on torch tensors, `impl="chunked"`: never materializes the full (N,V) logits.

Mirrors src/mlx_train_perf/core/chunked.py on torch: `streamed_lse_and_target` (:35-49),
`chunked_backward` (:52-90, fp32 d_hidden accumulator, g rounded to the weight dtype before
g @ w_chunk), `make_chunked_dense` (:93-132, recompute-lse backward, trainable head gradient) and
`make_chunked_quantized` (:135-183, chunk-sized dequantize). An explicit opt-in only; it runs with
torch ops on whatever device the tensors live on and is never chosen by `impl="auto"`.
"""
from __future__ import annotations

from collections.abc import Callable
from typing import NamedTuple

import torch

from mlx_train_perf.core.quant import dequantize


class QuantSpec(NamedTuple):
    """Frozen quantized head pieces (MLX affine layout; groups along D)."""
    w_q: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    group_size: int
    bits: int


MatmulChunk = Callable[[int, int], torch.Tensor]  # (v0, v1) -> (N, v1-v0) fp32 logits
WChunk = Callable[[int, int], torch.Tensor]       # (v0, v1) -> (v1-v0, D) weights

# Engagement counter (core/chunked.py:27-32): every custom backward increments its key first.
VJP_CALLS: dict[str, int] = {}


def streamed_lse_and_target(matmul_chunk: MatmulChunk, targets: torch.Tensor, *, v: int, chunk_size: int,
                            n: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Stream vocab chunks -> (lse (N,) fp32, target_logit (N,) fp32)."""
    dev = targets.device
    lse = torch.full((n,), float("-inf"), dtype=torch.float32, device=dev)
    tgt = torch.zeros((n,), dtype=torch.float32, device=dev)
    for v0 in range(0, v, chunk_size):
        v1 = min(v0 + chunk_size, v)
        logits = matmul_chunk(v0, v1)
        lse = torch.logaddexp(lse, torch.logsumexp(logits, dim=-1))
        in_chunk = (targets >= v0) & (targets < v1)
        idx = (targets - v0).clamp(0, v1 - v0 - 1)
        got = logits.gather(1, idx[:, None]).squeeze(1)
        tgt = torch.where(in_chunk, got, tgt)
    return lse, tgt


def chunked_backward(*, hidden: torch.Tensor, matmul_chunk: MatmulChunk, w_chunk: WChunk, targets: torch.Tensor,
                     lse: torch.Tensor, cotangent: torch.Tensor, v: int, chunk_size: int,
                     head_trainable: bool) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Given SAVED lse: d_hidden (hidden dtype) and d_w (or None if frozen)."""
    n, d = hidden.shape
    ct = cotangent.to(torch.float32)
    d_hidden32 = torch.zeros((n, d), dtype=torch.float32, device=hidden.device)
    d_w_chunks: list[torch.Tensor] = []
    for v0 in range(0, v, chunk_size):
        v1 = min(v0 + chunk_size, v)
        logits = matmul_chunk(v0, v1)
        p = torch.exp(logits - lse[:, None])
        onehot = torch.arange(v0, v1, device=hidden.device)[None, :] == targets[:, None]
        g32 = (p - onehot.to(p.dtype)) * ct[:, None]
        wc = w_chunk(v0, v1)
        g = g32.to(wc.dtype)
        d_hidden32 += (g @ wc).to(torch.float32)
        if head_trainable:
            d_w_chunks.append(g.T @ hidden)
    if not head_trainable:
        return d_hidden32.to(hidden.dtype), None
    return d_hidden32.to(hidden.dtype), torch.cat(d_w_chunks, dim=0)


class _ChunkedDense(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, w, targets, chunk_size):  # noqa: D401 -- torch signature
        n, v = hidden.shape[0], w.shape[0]

        def mm(v0: int, v1: int) -> torch.Tensor:
            return (hidden @ w[v0:v1].T).to(torch.float32)

        lse, tgt = streamed_lse_and_target(mm, targets, v=v, chunk_size=chunk_size, n=n)
        ctx.save_for_backward(hidden, w, targets)
        ctx.chunk_size = chunk_size
        return lse - tgt

    @staticmethod
    def backward(ctx, cotangent):
        VJP_CALLS["dense"] = VJP_CALLS.get("dense", 0) + 1
        hidden, w, targets = ctx.saved_tensors
        n, v = hidden.shape[0], w.shape[0]
        cs = ctx.chunk_size

        def mm(v0: int, v1: int) -> torch.Tensor:
            return (hidden @ w[v0:v1].T).to(torch.float32)

        lse, _ = streamed_lse_and_target(mm, targets, v=v, chunk_size=cs, n=n)
        d_hidden, d_w = chunked_backward(hidden=hidden, matmul_chunk=mm, w_chunk=lambda a, b: w[a:b],
                                         targets=targets, lse=lse, cotangent=cotangent, v=v, chunk_size=cs,
                                         head_trainable=ctx.needs_input_grad[1])
        return d_hidden, d_w, None, None


class _ChunkedQuant(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, targets, q, chunk_size):
        n, v = hidden.shape[0], q.w_q.shape[0]

        def mm(v0: int, v1: int) -> torch.Tensor:
            wc = dequantize(q.w_q[v0:v1], q.scales[v0:v1], q.biases[v0:v1], group_size=q.group_size,
                            bits=q.bits, dtype=hidden.dtype)
            return (hidden @ wc.T).to(torch.float32)

        lse, tgt = streamed_lse_and_target(mm, targets, v=v, chunk_size=chunk_size, n=n)
        ctx.save_for_backward(hidden, targets)
        ctx.q = q
        ctx.chunk_size = chunk_size
        return lse - tgt

    @staticmethod
    def backward(ctx, cotangent):
        VJP_CALLS["quantized"] = VJP_CALLS.get("quantized", 0) + 1
        hidden, targets = ctx.saved_tensors
        q, cs = ctx.q, ctx.chunk_size
        n, v = hidden.shape[0], q.w_q.shape[0]

        def w_chunk(v0: int, v1: int) -> torch.Tensor:  # chunk-sized dequant only
            return dequantize(q.w_q[v0:v1], q.scales[v0:v1], q.biases[v0:v1], group_size=q.group_size,
                              bits=q.bits, dtype=hidden.dtype)

        def mm(v0: int, v1: int) -> torch.Tensor:
            return (hidden @ w_chunk(v0, v1).T).to(torch.float32)

        lse, _ = streamed_lse_and_target(mm, targets, v=v, chunk_size=cs, n=n)
        d_hidden, _ = chunked_backward(hidden=hidden, matmul_chunk=mm, w_chunk=w_chunk, targets=targets, lse=lse,
                                       cotangent=cotangent, v=v, chunk_size=cs, head_trainable=False)
        return d_hidden, None, None, None


def make_chunked_dense(chunk_size: int) -> Callable[[torch.Tensor, torch.Tensor, torch.Tensor], torch.Tensor]:
    """Dense-head chunked CE. The head is an explicit input (its gradient flows if it requires grad)."""
    return lambda hidden, w, targets: _ChunkedDense.apply(hidden, w, targets, chunk_size)


def make_chunked_quantized(chunk_size: int, q: QuantSpec) -> Callable[[torch.Tensor, torch.Tensor], torch.Tensor]:
    """Quantized-head chunked CE: d_hidden only (the quantized head is frozen)."""
    return lambda hidden, targets: _ChunkedQuant.apply(hidden, targets, q, chunk_size)
