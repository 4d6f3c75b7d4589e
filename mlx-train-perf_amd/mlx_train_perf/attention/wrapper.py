"""`enable_flash_attention`: switch a torch causal-LM's attention onto `flash_attention`
(the torch counterpart of src/mlx_train_perf/attention/wrapper.py:205-292).

Two model shapes are served:

- **Hugging Face transformers models** (Llama / Qwen2 / Qwen3 / Mistral-style decoders): the
  attention implementation is registered in transformers' `AttentionInterface` (`IMPL_NAME`)
  and selected on the model config. Every decoder layer keeps its own projections, rotary
  embedding and (Qwen3) q/k norms; only the single attention call changes, exactly the seam the
  reference swaps (wrapper.py:126-157). A packed batch passes its `PackedMask` as the
  `mtp_segments=` keyword of the model call; transformers forwards it to every layer.
- **mlx-lm-style modules**: layers whose `self_attn` has `q_proj/k_proj/v_proj/o_proj`, a `rope`
  callable, `n_heads`, `n_kv_heads`, `scale` (and optionally `q_norm/k_norm`) are wrapped in
  `FlashAttentionWrapper`, which holds the original submodules under their original names (so
  LoRA injection by module path keeps working, wrapper.py:17-31) and reproduces the stock call.

Refusals (`UnsupportedAttentionError`, at enable time): sliding-window or mixed `layer_types`,
configured attention dropout, head_dim outside {64, 96, 128}, an unrecognised model shape.
There is no rate calibration on MI355X. With `seq_len` (and `batch_size`, `packed`) the launch
plan is validated up front (`plan/launch.py`), and a model already on the GPU runs one zeros
forward + backward at that shape, which loads the kernels a training step will launch.
"""
from __future__ import annotations

from typing import Any

import torch
from torch import nn

from mlx_train_perf.attention.api import flash_attention
from mlx_train_perf.attention.segments import PackedMask
from mlx_train_perf.errors import AttentionInputError, UnsupportedAttentionError
from mlx_train_perf.plan import launch as _plan

_KERNEL_HEAD_DIMS: tuple[int, ...] = (64, 96, 128)
IMPL_NAME = "mtp_hip_attention"  # no "flash" in the name: transformers routes such names to its kernel hub


def _resolve_mask(mask: Any) -> bool | PackedMask:
    """Map a caller's mask onto `flash_attention` (wrapper.py:72-96): "causal"/None -> causal,
    a PackedMask passes through, anything else (array / additive / sliding masks) is refused."""
    if isinstance(mask, PackedMask):
        return mask
    if isinstance(mask, str):
        if mask == "causal":
            return True
        raise AttentionInputError(
            f"unsupported string mask {mask!r}; the flash-attention training path only supports the 'causal' mask"
        )
    if mask is None:
        return True
    raise AttentionInputError(
        "array attention masks (sliding-window / additive) are not supported; the flash-attention training "
        "path is causal-only -- enable it only on full-attention models"
    )


class _UnsupportedMask:
    """What `_hf_mask` hands to the layers for a mask pattern the causal kernels cannot honour; the
    attention call then refuses with `reason` instead of silently attending causally."""

    __slots__ = ("reason",)

    def __init__(self, reason: str) -> None:
        self.reason = reason


def _hf_mask(batch_size: int, q_length: int, kv_length: int, q_offset: int = 0, kv_offset: int = 0,
             mask_function: Any = None, attention_mask: torch.Tensor | None = None, **kwargs: Any) -> Any:
    """transformers mask-interface function for IMPL_NAME.

    Returns None exactly when the layers may run plain causal attention: the pattern is the stock
    causal one and the 2-D padding mask is absent or all ones. A padding mask with a zero, or any
    other pattern (sliding window, packed sequences detected from `position_ids`, or/and overlays),
    comes back as an `_UnsupportedMask`, so `_hf_flash_attention` raises `AttentionInputError`."""
    from transformers.masking_utils import causal_mask_function  # noqa: PLC0415

    if mask_function is not None and mask_function is not causal_mask_function:
        return _UnsupportedMask(
            "the model requested a non-causal mask pattern (sliding window, packed position_ids or a mask "
            "overlay); the flash-attention path serves plain causal attention, or packed rows through "
            "`mtp_segments=`")
    if attention_mask is None:
        return None
    if attention_mask.dim() != 2:
        return _UnsupportedMask(f"a {attention_mask.dim()}-D attention mask was given")
    am = attention_mask[:, -kv_length:]
    if am.shape[1] == kv_length and bool(am.all()):
        return None
    return _UnsupportedMask("the batch has padding (attention_mask holds zeros); pack the rows or trim the padding")


def _hf_flash_attention(module: nn.Module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                        attention_mask: Any, scaling: float, dropout: float = 0.0,
                        mtp_segments: PackedMask | None = None, **kwargs: Any):
    """transformers attention-interface function: q (B,Hq,S,D), k/v (B,Hkv,S,D) post-RoPE;
    returns (output (B,S,Hq,D), None)."""
    if dropout:
        raise UnsupportedAttentionError("flash-attention training path does not support attention dropout")
    if attention_mask is not None:
        # `_hf_mask` returns None for every mask this path honours; anything else (padding, sliding
        # windows, packed position_ids, a prepared 4-D mask) is refused, with or without mtp_segments.
        reason = attention_mask.reason if isinstance(attention_mask, _UnsupportedMask) else \
            "an explicit attention mask was given"
        raise AttentionInputError(f"the flash-attention path cannot honour this mask: {reason}")
    impl = getattr(module.config, "_mtp_flash_impl", "auto")
    out = flash_attention(query, key, value, scale=float(scaling), causal=True, impl=impl, segments=mtp_segments)
    return out.transpose(1, 2).contiguous(), None


class FlashAttentionWrapper(nn.Module):
    """Drop-in replacement for an mlx-lm-style attention module (wrapper.py:99-157): original
    submodules held as direct attributes under their original names; only the attention call is
    swapped for `flash_attention`."""

    def __init__(self, original: nn.Module, *, impl: str) -> None:
        super().__init__()
        self.q_proj = original.q_proj
        self.k_proj = original.k_proj
        self.v_proj = original.v_proj
        self.o_proj = original.o_proj
        self.rope = original.rope
        self._has_qk_norm = hasattr(original, "q_norm")
        if self._has_qk_norm:
            self.q_norm = original.q_norm
            self.k_norm = original.k_norm
        self.n_heads = original.n_heads
        self.n_kv_heads = original.n_kv_heads
        self.scale = original.scale
        self._impl = impl

    def forward(self, x: torch.Tensor, mask: Any = None, cache: Any = None) -> torch.Tensor:
        if cache is not None:
            raise AttentionInputError("FlashAttentionWrapper is a training-only path; a KV cache is not supported")
        b, length, _ = x.shape
        queries, keys, values = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        queries = queries.reshape(b, length, self.n_heads, -1)
        keys = keys.reshape(b, length, self.n_kv_heads, -1)
        if self._has_qk_norm:
            queries = self.q_norm(queries)
            keys = self.k_norm(keys)
        queries = queries.transpose(1, 2)
        keys = keys.transpose(1, 2)
        values = values.reshape(b, length, self.n_kv_heads, -1).transpose(1, 2)
        queries = self.rope(queries)
        keys = self.rope(keys)
        resolved = _resolve_mask(mask)
        segments = resolved if isinstance(resolved, PackedMask) else None
        out = flash_attention(queries, keys, values, scale=self.scale, causal=True, segments=segments,
                              impl=self._impl)  # type: ignore[arg-type]
        return self.o_proj(out.transpose(1, 2).reshape(b, length, -1))


def _config_of(model: Any) -> Any:
    return getattr(model, "config", None) or getattr(model, "args", None)


def _head_dim(cfg: Any) -> int:
    hd = getattr(cfg, "head_dim", None)
    if hd:
        return int(hd)
    return int(cfg.hidden_size // cfg.num_attention_heads)


def _refusals(cfg: Any, layers: Any) -> int:
    layer_types = getattr(cfg, "layer_types", None)
    if layer_types is not None:
        offending = sorted({lt for lt in layer_types if lt != "full_attention"})
        if offending:
            raise UnsupportedAttentionError(
                f"enable_flash_attention supports full-attention models only; model declares non-full-attention "
                f"layer_types {offending} -- sliding-window / mixed attention is out of scope"
            )
    if getattr(cfg, "use_sliding_window", False) or any(getattr(layer, "use_sliding", False) for layer in layers):
        raise UnsupportedAttentionError(
            "enable_flash_attention supports full-attention models only; model has sliding-window attention"
        )
    dropout = getattr(cfg, "attention_dropout", 0.0)
    if dropout:
        raise UnsupportedAttentionError(
            f"enable_flash_attention does not support attention dropout (attention_dropout={dropout}); it must be 0"
        )
    head_dim = _head_dim(cfg)
    if head_dim not in _KERNEL_HEAD_DIMS:
        raise UnsupportedAttentionError(
            f"enable_flash_attention supports head_dim in {_KERNEL_HEAD_DIMS}; model has head_dim={head_dim}"
        )
    return head_dim


def _model_device_dtype(model: Any) -> tuple[torch.device, torch.dtype] | None:
    for p in model.parameters():
        if p.is_floating_point():
            return p.device, p.dtype
    return None


def _prewarm(model: Any, *, impl: str, seq_len: int, batch_size: int, hq: int, hkv: int, head_dim: int,
             packed: bool) -> None:
    """One zeros forward + backward at the training shape (the counterpart of the reference's
    `_prewarm_rate_caches`, wrapper.py:170-202), so the first training step does not pay for loading
    the kernels' code objects; with `packed`, a second one with a single-segment `PackedMask`, which
    runs the packed instantiations and the backward's work-order sort. A model on the CPU skips it
    (there is nothing to load), as does a dtype the kernels do not take."""
    where = _model_device_dtype(model)
    if where is None or where[0].type != "cuda" or where[1] not in (torch.bfloat16, torch.float32):
        return
    dev, dt = where
    q = torch.zeros((batch_size, hq, seq_len, head_dim), dtype=dt, device=dev, requires_grad=True)
    k = torch.zeros((batch_size, hkv, seq_len, head_dim), dtype=dt, device=dev, requires_grad=True)
    v = torch.zeros((batch_size, hkv, seq_len, head_dim), dtype=dt, device=dev, requires_grad=True)
    masks: list[PackedMask | None] = [None]
    if packed:
        z = torch.zeros((batch_size, seq_len), dtype=torch.int32, device=dev)
        masks.append(PackedMask(seg_id=z, seg_start=z))
    for seg in masks:
        out = flash_attention(q, k, v, scale=1.0 / head_dim ** 0.5, causal=True, impl=impl, segments=seg)  # type: ignore[arg-type]
        out.backward(torch.zeros_like(out))


def enable_flash_attention(model: Any, *, impl: str = "auto", seq_len: int | None = None, batch_size: int = 1,
                           packed: bool = False) -> None:
    """Enable the flash-attention training path on `model` in place (wrapper.py:205-292).

    `impl`: forwarded to `flash_attention` per call ("auto"/"kernel" -> HIP kernels,
    "reference" -> the materialized oracle, small shapes only). `seq_len`/`batch_size`: when given
    with a kernel impl, the launch plan for that shape is computed now, so an unsupported shape fails
    at enable time, and a model already on the GPU in bf16 or fp32 runs one zeros forward + backward at that
    shape (`packed=True`: also one with a single-segment `PackedMask`, the packed kernels a
    `mtp_segments=` / `PackedMask` step will launch), as the reference pre-warms its rate caches."""
    cfg = _config_of(model)
    inner = getattr(model, "model", None)
    layers = getattr(inner, "layers", None)
    if cfg is None or layers is None:
        raise UnsupportedAttentionError(
            f"unsupported model architecture {type(model).__name__!r}: expected a causal LM with "
            "`.model.layers` and a config"
        )
    _refusals(cfg, layers)
    first = layers[0].self_attn
    if hasattr(cfg, "_attn_implementation") and not hasattr(first, "rope"):
        from transformers import AttentionInterface  # noqa: PLC0415 -- only for transformers models

        AttentionInterface.register(IMPL_NAME, _hf_flash_attention)
        try:
            from transformers import AttentionMaskInterface  # noqa: PLC0415

            AttentionMaskInterface.register(IMPL_NAME, _hf_mask)
        except ImportError:
            pass
        cfg._mtp_flash_impl = impl
        if hasattr(model, "set_attn_implementation"):
            model.set_attn_implementation(IMPL_NAME)
        else:
            cfg._attn_implementation = IMPL_NAME
    else:
        for layer in layers:
            if not isinstance(layer.self_attn, FlashAttentionWrapper):
                layer.self_attn = FlashAttentionWrapper(layer.self_attn, impl=impl)
    if seq_len is not None and impl in ("auto", "kernel"):
        hq = int(cfg.num_attention_heads)
        hkv = int(getattr(cfg, "num_key_value_heads", hq) or hq)
        if hq % hkv:
            raise UnsupportedAttentionError(f"Hq={hq} must be a multiple of Hkv={hkv}")
        head_dim = _head_dim(cfg)
        _plan.attn_plan(b=batch_size, hq=hq, hkv=hkv, s=seq_len, dh=head_dim)
        _prewarm(model, impl=impl, seq_len=seq_len, batch_size=batch_size, hq=hq, hkv=hkv, head_dim=head_dim,
                 packed=packed)


def is_enabled(model: Any) -> bool:
    cfg = _config_of(model)
    if cfg is not None and getattr(cfg, "_attn_implementation", None) == IMPL_NAME:
        return True
    layers = getattr(getattr(model, "model", None), "layers", None) or []
    return bool(layers) and all(isinstance(layer.self_attn, FlashAttentionWrapper) for layer in layers)
