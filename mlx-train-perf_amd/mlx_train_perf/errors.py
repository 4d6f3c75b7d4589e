"""Typed error hierarchy, same names and meaning as the reference (src/mlx_train_perf/errors.py:1-76).

Only the errors the hot path raises are defined; each keeps the reference's semantics:
no silent fallback, refuse before launch.
"""


class MlxTrainPerfError(Exception):
    """Root of all mlx-train-perf errors."""


class UnsupportedHeadError(MlxTrainPerfError):
    """Head kind/dtype the requested impl cannot serve (no silent fallback)."""


class LaunchBudgetError(MlxTrainPerfError):
    """A launch would exceed its workspace budget; refused before launch.

    (The reference raises it for the macOS GPU-watchdog budget, errors.py:13-14; on MI355X the only
    budget is the caller-provided workspace.)"""


class LossInputError(MlxTrainPerfError):
    """Shape/dtype/target-range validation failure at the loss boundary."""


class PlanInputError(MlxTrainPerfError):
    """Shape/config validation failure in the memory planner."""


class DoesNotFitError(MlxTrainPerfError):
    """Planner verdict: predicted peak exceeds the memory budget."""


class AdapterError(MlxTrainPerfError):
    """The model cannot be split into trunk + head (unsupported architecture, missing modules)."""


class MissingDependencyError(MlxTrainPerfError):
    """A required native component (the HIP extension) or optional dependency is absent."""


class UnsupportedAttentionError(MlxTrainPerfError):
    """Attention impl/config combination the requested impl cannot serve (no silent fallback) --
    e.g. an unsupported dtype, head_dim, or causal=False for impl='kernel'."""


class AttentionInputError(MlxTrainPerfError):
    """Shape validation failure at the flash_attention boundary (non-4D tensors, Hq not a
    multiple of Hkv, mismatched N/D/batch across q/k/v)."""


class PackingError(MlxTrainPerfError):
    """Sequence-packing input validation failure (empty dataset, zero-length sequence,
    non-positive pack_len) -- no silent fallback."""
