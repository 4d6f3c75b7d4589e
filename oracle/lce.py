"""CPU restatement of the reference's linear cross-entropy oracle (test infrastructure only).

Follows:
- src/mlx_train_perf/core/naive.py:9-14 (`naive_linear_ce`): fp32 logits = hidden @ w.T,
  lse = logsumexp, tgt = logits[i, y_i], nll = lse - tgt; the parity convention is the fp32-upcast
  inputs (tests/test_kernel_parity.py:34).
- src/mlx_train_perf/core/chunked.py:35-49 (`streamed_lse_and_target`): chunked lse/tgt.
- src/mlx_train_perf/core/chunked.py:52-90 (`chunked_backward`): d_hidden = sum over vocab chunks of
  g @ w_chunk with g = (exp(logits - lse) - onehot) * ct, g rounded to the weight dtype before the
  product (chunked.py:84-86), fp32 accumulation.

Every function runs on the device its inputs live on (CPU here; the GPU parity tests run it in fp64
on the GPU for the flagship shapes).

The ignore_index contract of this build (the reference masks in its trainer adapter,
adapters/mlx_lm.py:206-216): rows whose target equals ignore_index get nll = 0, tgt = 0, a zero
gradient row, and are excluded from the mean.
"""
from __future__ import annotations

import torch


def _bf16_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(x.dtype)


def naive_linear_ce(hidden: torch.Tensor, w: torch.Tensor, targets: torch.Tensor,
                    dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """(N,D) x (V,D) -> per-token NLL (N,), materializing the full (N,V) logits
    (core/naive.py:9-14). Inputs are upcast to `dtype` first."""
    logits = hidden.to(dtype) @ w.to(dtype).T
    lse = torch.logsumexp(logits, dim=-1)
    tgt = logits.gather(1, targets.long()[:, None]).squeeze(1)
    return lse - tgt


def forward(hidden: torch.Tensor, w: torch.Tensor, targets: torch.Tensor, *, ignore_index: int = -100,
            chunk: int = 8192, dtype: torch.dtype = torch.float64) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(nll, lse, tgt), each (N,) in `dtype`, streamed over vocab chunks
    (core/chunked.py:35-49) so the (N,V) logits never exist at once.

    Ignored rows: nll = 0, tgt = 0, lse computed normally. A target outside [0, V) that is not
    ignore_index keeps tgt = 0 (nll = lse), matching the reference kernel with
    validate_targets=False (core/kernel/source.py:46,143-144)."""
    n = hidden.shape[0]
    v = w.shape[0]
    h = hidden.to(dtype)
    y = targets.long()
    lse = torch.full((n,), float("-inf"), dtype=dtype, device=hidden.device)
    tgt = torch.zeros((n,), dtype=dtype, device=hidden.device)
    for v0 in range(0, v, chunk):
        v1 = min(v0 + chunk, v)
        logits = h @ w[v0:v1].to(dtype).T
        lse = torch.logaddexp(lse, torch.logsumexp(logits, dim=-1))
        in_chunk = (y >= v0) & (y < v1)
        idx = (y - v0).clamp(0, v1 - v0 - 1)
        got = logits.gather(1, idx[:, None]).squeeze(1)
        tgt = torch.where(in_chunk, got, tgt)
    ignored = y == ignore_index
    tgt = torch.where(ignored, torch.zeros_like(tgt), tgt)
    nll = torch.where(ignored, torch.zeros_like(lse), lse - tgt)
    return nll, lse, tgt


def backward(hidden: torch.Tensor, w: torch.Tensor, targets: torch.Tensor, lse: torch.Tensor,
             cotangent: torch.Tensor, *, ignore_index: int = -100, round_g_bf16: bool = True,
             chunk: int = 8192, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """d_hidden (N,D) in `dtype` from the saved lse (core/chunked.py:52-90).

    g = (exp(logits - lse) - onehot) * ct per vocab chunk; when `round_g_bf16` g is rounded to bf16
    before g @ w_chunk, as the reference does for a bf16 head (chunked.py:84-86); accumulation is in
    `dtype`. Ignored rows get ct = 0."""
    n, d = hidden.shape
    v = w.shape[0]
    h = hidden.to(dtype)
    y = targets.long()
    ct = torch.where(y == ignore_index, torch.zeros_like(cotangent, dtype=dtype), cotangent.to(dtype))
    lse_ = lse.to(dtype)
    dh = torch.zeros((n, d), dtype=dtype, device=hidden.device)
    for v0 in range(0, v, chunk):
        v1 = min(v0 + chunk, v)
        wc = w[v0:v1].to(dtype)
        logits = h @ wc.T
        p = torch.exp(logits - lse_[:, None])
        onehot = (torch.arange(v0, v1, device=hidden.device)[None, :] == y[:, None]).to(dtype)
        g = (p - onehot) * ct[:, None]
        if round_g_bf16:
            g = _bf16_round(g)
        dh += g @ wc
    return dh


def backward_dw(hidden: torch.Tensor, w: torch.Tensor, targets: torch.Tensor, lse: torch.Tensor,
                cotangent: torch.Tensor, *, ignore_index: int = -100, round_g_bf16: bool = True, chunk: int = 8192,
                dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """d_w (V,D) of a trainable head: per vocab chunk g.T @ hidden (core/chunked.py:87-90), with the
    same g as `backward`."""
    v = w.shape[0]
    h = hidden.to(dtype)
    y = targets.long()
    ct = torch.where(y == ignore_index, torch.zeros_like(cotangent, dtype=dtype), cotangent.to(dtype))
    out = torch.empty((v, hidden.shape[1]), dtype=dtype, device=hidden.device)
    for v0 in range(0, v, chunk):
        v1 = min(v0 + chunk, v)
        wc = w[v0:v1].to(dtype)
        p = torch.exp(h @ wc.T - lse.to(dtype)[:, None])
        onehot = (torch.arange(v0, v1, device=hidden.device)[None, :] == y[:, None]).to(dtype)
        g = (p - onehot) * ct[:, None]
        if round_g_bf16:
            g = _bf16_round(g)
        out[v0:v1] = g.T @ h
    return out


def reduce_mean(nll: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100) -> torch.Tensor:
    """Mean over non-ignored rows (the adapter's (nll * mask).sum() / ntoks, adapters/mlx_lm.py:212-216);
    0 when every row is ignored. Pinned by a hand-computed case in tests/test_oracle_lce.py."""
    valid = targets.long() != ignore_index
    return nll[valid].sum() / valid.sum().clamp(min=1)
