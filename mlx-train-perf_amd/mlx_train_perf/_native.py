"""ctypes binding of the HIP C-ABI library (``libmtp_hip.so``, declared in ``include/mtp_hip.h``).

This is the only place the package touches native code. The library is built in-tree by
``__graft_entry__.build()`` (or ``python -m mlx_train_perf._build``) for gfx950. There is no fallback:
if the library is missing or no GPU is visible, the kernel impls raise ``MissingDependencyError`` /
``UnsupportedHeadError`` / ``UnsupportedAttentionError`` before any launch.

torch must be imported before the library is loaded so that the process holds exactly one HIP
runtime (torch's): the library's ``libamdhip64.so.7`` dependency then resolves to the copy torch
already mapped, and torch's stream handles are valid for our launches.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

from mlx_train_perf.errors import (
    AttentionInputError,
    LaunchBudgetError,
    LossInputError,
    MissingDependencyError,
    MlxTrainPerfError,
    UnsupportedAttentionError,
    UnsupportedHeadError,
)

LIB_NAME = "libmtp_hip.so"
LIB_PATH = Path(os.environ.get("MTP_HIP_LIB", str(Path(__file__).resolve().parent / LIB_NAME)))

ABI_VERSION = 5
MTP_OK = 0
MTP_ERR_INPUT = -1
MTP_ERR_UNSUPPORTED = -2
MTP_ERR_WORKSPACE = -3
MTP_ERR_RUNTIME = -4

HEAD_DENSE = 0
HEAD_Q4 = 1
HEAD_Q4_STAGED = 2      # kinds that stage the head chunk-wise in the workspace: the backward each
HEAD_DENSE_STAGED = 3   # transposed (4-bit: dequantized) vocab chunk instead of a cached transposed
                        # copy, the 4-bit forward runs of vocab splits dequantized to rows

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_size = ctypes.c_size_t

# name -> (restype, argtypes); the single source of truth for the Python side of the ABI.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "mtp_last_error": (ctypes.c_char_p, []),
    "mtp_abi_version": (ctypes.c_int, []),
    "mtp_lce_fwd_workspace_bytes": (_size, [_i64, _i64, _i64, _i32]),
    "mtp_lce_fwd_stage_workspace_bytes": (_size, [_i64, _i64, _i64, _size]),
    "mtp_lce_fwd": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _i64, _i64, _i64, _i32, _i64, _c_void_p, _c_void_p, _c_void_p,
                                   _c_void_p, _size, _c_void_p]),
    "mtp_lce_fwd_noalloc": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                           _i64, _i64, _i64, _i32, _i64, _c_void_p, _c_void_p, _c_void_p,
                                           _c_void_p]),
    "mtp_lce_fwd_noalloc_max_workspace_bytes": (_size, []),
    "mtp_lce_bwd_row_block": (_i64, [_i64, _i64, _i64, _size]),
    "mtp_lce_bwd_chunk": (_i64, [_i64, _i64, _i64, _size]),
    "mtp_lce_bwd_stage_chunk": (_i64, [_i64, _i64, _i64, _i32, _size]),
    "mtp_lce_bwd_workspace_bytes": (_size, [_i64, _i64, _i64, _i32, _i64, _i64]),
    "mtp_lce_head_t_ld": (_i64, [_i64]),
    "mtp_lce_head_transpose": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32,
                                              _c_void_p, _c_void_p]),
    "mtp_lce_bwd": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _i64, _i64, _i64, _i32, _i64, _c_void_p, _c_void_p, _c_void_p,
                                   _c_void_p, _i64, _i64, _c_void_p, _size, _c_void_p]),
    "mtp_attn_fwd": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64,
                                    _f32, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "mtp_attn_bwd_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "mtp_attn_bwd_dkv_splits": (ctypes.c_int, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "mtp_bench_mfma_ceiling": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _c_void_p, _c_void_p]),
    "mtp_attn_bwd": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                    _i64, _i64, _i64, _i64, _i64, _f32, _i32, _c_void_p, _c_void_p,
                                    _c_void_p, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    # fp32 inputs
    "mtp_lce_fwd_f32_workspace_bytes": (_size, [_i64, _i64, _i64, _i32]),
    "mtp_lce_fwd_f32": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                       _i64, _i64, _i64, _i32, _i64, _c_void_p, _c_void_p, _c_void_p,
                                       _c_void_p, _size, _c_void_p]),
    "mtp_lce_bwd_f32_chunk": (_i64, [_i64, _i64, _i64, _size]),
    "mtp_lce_bwd_f32_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "mtp_lce_bwd_f32": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                       _i64, _i64, _i64, _i32, _i64, _c_void_p, _c_void_p, _c_void_p,
                                       _c_void_p, _i64, _c_void_p, _size, _c_void_p]),
    "mtp_attn_fwd_f32": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64,
                                        _f32, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "mtp_attn_bwd_f32_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "mtp_attn_bwd_f32": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                        _i64, _i64, _i64, _i64, _i64, _f32, _i32, _c_void_p, _c_void_p,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library with typed signatures; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise MissingDependencyError(
                f"HIP extension {LIB_PATH} is not built; run `python -c \"import __graft_entry__ as g; "
                "g.build()\"` from the repository root (hipcc --offload-arch=gfx950)."
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.mtp_abi_version() != ABI_VERSION:
            raise MissingDependencyError(f"{LIB_PATH} has ABI version {lib.mtp_abi_version()}, expected "
                                         f"{ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def gpu_available() -> bool:
    return torch.cuda.is_available()


def last_error() -> str:
    msg = load().mtp_last_error()
    return msg.decode() if msg else ""


_ERR_LOSS = {MTP_ERR_INPUT: LossInputError, MTP_ERR_UNSUPPORTED: UnsupportedHeadError,
             MTP_ERR_WORKSPACE: LaunchBudgetError}
_ERR_ATTN = {MTP_ERR_INPUT: AttentionInputError, MTP_ERR_UNSUPPORTED: UnsupportedAttentionError,
             MTP_ERR_WORKSPACE: LaunchBudgetError}


def check(rc: int, *, domain: str) -> None:
    """Map a negative C-ABI return code onto the reference's typed exceptions."""
    if rc == MTP_OK:
        return
    table = _ERR_LOSS if domain == "loss" else _ERR_ATTN
    exc = table.get(rc, MlxTrainPerfError)
    raise exc(last_error() or f"mtp call failed with code {rc}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def on_device(t: torch.Tensor):
    """Context that makes t's GPU the current device for a C-ABI call. The launches go to t's stream;
    HIP calls inside the library that act on the current device (the no-allocation forward's scratch
    lookup, error queries) then see the same device whatever the caller had current."""
    return torch.cuda.device(t.device)
