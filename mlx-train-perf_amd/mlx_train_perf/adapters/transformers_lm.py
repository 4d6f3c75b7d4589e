"""Trainer adapter for torch causal LMs: `split_model`, `make_loss_fn`, `make_packed_loss_fn`
(the torch counterpart of src/mlx_train_perf/adapters/mlx_lm.py:140-297).

Loss contract (the mlx-lm trainer's `default_loss`, quoted at adapters/mlx_lm.py:5-20):
inputs = batch[:, :-1], targets = batch[:, 1:], steps = 1..T, mask = (steps >= lengths[:, 0]) &
(steps <= lengths[:, 1]), loss = (nll * mask).sum() / ntoks, returning (loss, ntoks).
The fused loss replaces the `(B, T, V)` logits: the model's trunk produces hidden states and
`linear_cross_entropy(..., reduction="none")` the per-token NLL. This contract is only available
as documented text (mlx-lm is not installed), so its numerics are checked against a plain torch
restatement of that formula, not against mlx-lm itself.

Supported models: Hugging Face transformers causal LMs with `.model` (trunk returning
`last_hidden_state`) and `.lm_head` (`nn.Linear`), or tied word embeddings
(`config.tie_word_embeddings`). The head and its `trainable` flag are re-read from the live model
on every call (adapters/mlx_lm.py:22-33: a construction-time snapshot would go stale).
"""
from __future__ import annotations

from collections.abc import Callable
from typing import Any, Literal

import torch
from torch import nn

from mlx_train_perf.attention.segments import PackedMask
from mlx_train_perf.core.loss import DenseHead, HeadRef, linear_cross_entropy, resolve_impl, tied_head
from mlx_train_perf.errors import AdapterError

_Impl = Literal["auto", "kernel", "chunked", "naive"]


def _head_from_linear(module: nn.Module) -> DenseHead:
    if not isinstance(module, nn.Linear):
        raise AdapterError(f"unsupported head module type {type(module).__name__!r}; expected nn.Linear")
    if module.bias is not None:
        raise AdapterError("lm_head with a bias is not supported by the fused loss")
    return DenseHead(weight=module.weight, trainable=module.weight.requires_grad)


def split_model(model: Any) -> tuple[Callable[..., torch.Tensor], HeadRef]:
    """(trunk, head): trunk(input_ids, **kw) -> hidden (B, T, D); head from lm_head or tied embeddings."""
    inner = getattr(model, "model", None)
    if inner is None or not hasattr(inner, "layers"):
        raise AdapterError(f"unsupported model architecture {type(model).__name__!r}: expected `.model.layers`")

    def trunk(x: torch.Tensor, **kw: Any) -> torch.Tensor:
        out = inner(input_ids=x, **kw)
        return out.last_hidden_state if hasattr(out, "last_hidden_state") else out

    cfg = getattr(model, "config", None)
    if cfg is not None and getattr(cfg, "tie_word_embeddings", False):
        emb = inner.embed_tokens
        return trunk, tied_head(emb.weight, trainable=emb.weight.requires_grad)
    head = getattr(model, "lm_head", None)
    if head is None:
        raise AdapterError("model has neither an lm_head nor tied word embeddings")
    return trunk, _head_from_linear(head)


def make_loss_fn(model: Any, *, impl: _Impl = "auto",
                 allow_unverified_mlx: bool = False) -> Callable[[Any, torch.Tensor, torch.Tensor], tuple[torch.Tensor, torch.Tensor]]:
    """`loss(model, batch, lengths) -> (loss, ntoks)` with the mlx-lm trainer's mask and
    normalization (adapters/mlx_lm.py:167-218). `lengths` is (B, 2) int: (offset, length)."""
    split_model(model)  # fail fast; re-derived per call
    resolved: dict[str, str] = {}

    def loss_fn(model_arg: Any, batch: torch.Tensor, lengths: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        trunk, head = split_model(model_arg)
        inputs, targets = batch[:, :-1], batch[:, 1:]
        hidden = trunk(inputs)
        if "impl" not in resolved:
            n = hidden.shape[0] * hidden.shape[1]
            resolved["impl"] = resolve_impl(head=head, dtype=hidden.dtype, n=n, impl=impl,
                                            allow_unverified_mlx=allow_unverified_mlx).impl
        nll = linear_cross_entropy(hidden, head, targets, impl=resolved["impl"], reduction="none",
                                   validate_targets=False)
        steps = torch.arange(1, targets.shape[1] + 1, device=targets.device)
        mask = (steps >= lengths[:, 0:1]) & (steps <= lengths[:, 1:])
        ntoks = mask.sum()
        loss = (nll * mask).to(torch.float32).sum() / ntoks
        return loss, ntoks

    return loss_fn


def make_packed_loss_fn(model: Any, *, impl: _Impl = "auto", allow_unverified_mlx: bool = False):
    """`loss(model, batch, seg_id, seg_start, loss_mask) -> (loss, ntoks)` for packed rows
    (adapters/mlx_lm.py:221-297): the PackedMask is threaded to every attention call, the loss is
    normalized by `loss_mask`. Requires `enable_flash_attention(model)` first (AdapterError)."""
    from mlx_train_perf.attention.wrapper import is_enabled  # noqa: PLC0415

    split_model(model)
    if not is_enabled(model):
        raise AdapterError("make_packed_loss_fn requires enable_flash_attention(model) first")
    resolved: dict[str, str] = {}

    def loss_fn(model_arg: Any, batch: torch.Tensor, seg_id: torch.Tensor, seg_start: torch.Tensor,
                loss_mask: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        trunk, head = split_model(model_arg)
        inputs, targets = batch[:, :-1], batch[:, 1:]
        pm = PackedMask(seg_id=seg_id, seg_start=seg_start)
        hidden = trunk(inputs, mtp_segments=pm)
        if "impl" not in resolved:
            n = hidden.shape[0] * hidden.shape[1]
            resolved["impl"] = resolve_impl(head=head, dtype=hidden.dtype, n=n, impl=impl,
                                            allow_unverified_mlx=allow_unverified_mlx).impl
        nll = linear_cross_entropy(hidden, head, targets, impl=resolved["impl"], reduction="none",
                                   validate_targets=False)
        ntoks = loss_mask.sum()
        loss = (nll * loss_mask).to(torch.float32).sum() / ntoks
        return loss, ntoks

    return loss_fn
