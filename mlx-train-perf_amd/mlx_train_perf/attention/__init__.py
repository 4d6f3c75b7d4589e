"""Flash attention API and oracles -- re-exports (mirror of src/mlx_train_perf/attention/__init__.py)."""
from mlx_train_perf.attention.api import flash_attention, resolve_attention_impl
from mlx_train_perf.attention.reference import flash_attention_reference, kv_head_for, math_attention
from mlx_train_perf.attention.segments import PackedMask, segment_allowed
from mlx_train_perf.attention.wrapper import FlashAttentionWrapper, enable_flash_attention

__all__ = [
    "FlashAttentionWrapper",
    "PackedMask",
    "enable_flash_attention",
    "flash_attention",
    "flash_attention_reference",
    "kv_head_for",
    "math_attention",
    "resolve_attention_impl",
    "segment_allowed",
]
