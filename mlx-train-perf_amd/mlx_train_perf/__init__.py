"""mlx-train-perf hot path for AMD MI355X (gfx950): fused linear cross-entropy and flash attention.

Same public names as the reference package (src/mlx_train_perf/__init__.py:1-12); tensors are torch
tensors and the kernel impls run hand-written HIP through the C-ABI library libmtp_hip.so.
"""
from mlx_train_perf.core.loss import (
    DenseHead,
    HeadRef,
    QuantizedHead,
    Resolution,
    linear_cross_entropy,
    resolve_impl,
    tied_head,
)

__all__ = ["DenseHead", "HeadRef", "QuantizedHead", "Resolution", "linear_cross_entropy",
           "resolve_impl", "tied_head"]
