"""`impl="naive"`: the loss computed from the whole logits matrix.

This is the baseline the fused kernels are measured against: it forms all N x V logits at once
(4.98 GB in fp32 at N=8192, V=151936), which is exactly the allocation the fused path avoids. The
arithmetic follows src/mlx_train_perf/core/naive.py:9-14: the product in the inputs' dtype, then
fp32 for the log-sum-exp and the target pick. An explicit opt-in only; `impl="auto"` never picks it.
"""
import torch


def naive_linear_ce(hidden: torch.Tensor, w: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Per-row NLL, fp32 of shape (N,), of hidden (N, D) against head w (V, D) and integer targets
    (N,) in [0, V): logsumexp of the row's logits minus its target logit, with every logit held in
    memory at once."""
    logits = (hidden @ w.T).to(torch.float32)
    lse = torch.logsumexp(logits, dim=-1)
    tgt = logits.gather(1, targets.long()[:, None]).squeeze(1)
    return lse - tgt
