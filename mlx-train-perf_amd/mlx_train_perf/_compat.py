"""Device gate for the kernel impls: the MI355X analogue of the reference's verified-mlx gate
(src/mlx_train_perf/_compat.py:6-24). The HIP code objects are built for gfx950 only, so the kernel
impls refuse, with the caller's typed error, a tensor that is not on a GPU or a GPU of another
architecture (unless `allow_unverified=True`), instead of failing inside a launch.
"""
from __future__ import annotations

import torch

VERIFIED_ARCHS = ("gfx950",)


def device_arch(device: torch.device | int | None = None) -> str:
    props = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
    return getattr(props, "gcnArchName", "").split(":")[0]


def check_device_verified(*, allow_unverified: bool, error: type[Exception]) -> None:
    if not torch.cuda.is_available():
        raise error("kernel impl requires an MI355X (gfx950) GPU; none is visible. Use impl='chunked' / "
                    "impl='reference' on CPU.")
    if allow_unverified:
        return
    arch = device_arch()
    if arch not in VERIFIED_ARCHS:
        raise error(f"kernel impl is built for {VERIFIED_ARCHS}; device reports {arch!r} "
                    "(pass allow_unverified_mlx=True to try anyway)")


def require_gpu_tensor(t: torch.Tensor, *, error: type[Exception]) -> None:
    if t.device.type != "cuda":
        raise error(f"kernel impl needs GPU tensors (got a tensor on {t.device})")
