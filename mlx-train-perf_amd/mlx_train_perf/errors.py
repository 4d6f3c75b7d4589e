"""Exceptions of this package. The class names and the hierarchy are those of the reference
(src/mlx_train_perf/errors.py:1-76), so callers can catch the same types; only the errors the hot
path can raise are defined. Every refusal happens on the host, before anything is launched.
"""


class MlxTrainPerfError(Exception):
    """Base class: catching it catches every error this package raises on purpose."""


class UnsupportedHeadError(MlxTrainPerfError):
    """The requested loss impl cannot serve this head kind or dtype. The message names the impl that
    can; nothing switches impls behind the caller's back."""


class LaunchBudgetError(MlxTrainPerfError):
    """A launch was refused because its workspace is missing or smaller than the plan needs.

    (The reference uses this type for its macOS GPU-watchdog time budget, errors.py:13-14; compute
    queues on MI355X have no such watchdog, so the workspace is the only budget left.)"""


class LossInputError(MlxTrainPerfError):
    """The loss was called with inconsistent shapes, a wrong dtype, or targets outside [0, V)."""


class PlanInputError(MlxTrainPerfError):
    """The memory planner was given a shape or config it cannot price (e.g. an unknown dtype)."""


class DoesNotFitError(MlxTrainPerfError):
    """The memory planner predicts a peak above the memory available for the run."""


class AdapterError(MlxTrainPerfError):
    """The model does not split into a trunk and a head the fused loss can use (unknown
    architecture, missing modules, a head with a bias)."""


class MissingDependencyError(MlxTrainPerfError):
    """Something required is absent: the built HIP library, or an optional Python package."""


class UnsupportedAttentionError(MlxTrainPerfError):
    """The requested attention impl cannot serve this configuration (dtype, head_dim, mask). The
    message names the impl that can."""


class AttentionInputError(MlxTrainPerfError):
    """flash_attention was called with malformed inputs: tensors that are not 4-D, Hq not a multiple
    of Hkv, disagreeing batch / length / head_dim, tensors on different devices, or a segment layout
    that breaks the packed-row contract."""


class PackingError(MlxTrainPerfError):
    """The sequence packer was given unusable input: no sequences, an empty sequence, or a
    non-positive pack length."""
