"""Full-materialization loss (the memory spike the library exists to remove), `impl="naive"`.

Mirrors src/mlx_train_perf/core/naive.py:9-14 on torch tensors: logits = hidden @ w.T in the
input dtype, cast to fp32, logsumexp minus the target logit. An explicit opt-in only; never chosen
by `impl="auto"`.
"""
import torch


def naive_linear_ce(hidden: torch.Tensor, w: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """(N,D) x (V,D) -> per-token NLL (N,), float32. Materializes full (N,V) logits."""
    logits = (hidden @ w.T).to(torch.float32)
    lse = torch.logsumexp(logits, dim=-1)
    tgt = logits.gather(1, targets.long()[:, None]).squeeze(1)
    return lse - tgt
