"""Public loss API: HeadRef seam, impl resolution, autograd wiring (mirror of
src/mlx_train_perf/core/loss.py on torch tensors).

Residual contract (loss.py:1-7): the kernel autograd Function returns (nll_rows, lse, tgt); only
`lse` is saved for the backward; this public wrapper consumes nll_rows and applies `reduction`
outside the Function. Aux outputs never leak.

MI355X specifics:
- `impl="kernel"` (and `"auto"`) runs the HIP kernels of libmtp_hip.so: the logit-free forward and
  the chunked-recompute dL/dH backward. Hidden states (and a dense head) are bf16 (bf16 MFMA,
  fp32 accumulation) or fp32 (fp32 MFMA, fp32 gradients), on a gfx950 device.
- `ignore_index` (default -100): ignored rows get nll = 0, a zero gradient, and are excluded from
  `reduction="mean"`, which is exactly the trainer adapter's `(nll * mask).sum() / ntoks`
  (adapters/mlx_lm.py:212-216). With no ignored rows every reduction equals the reference's.
- No silent fallback: an unsupported config raises the reference's typed errors.
"""
from __future__ import annotations

import os
import threading
import weakref
from dataclasses import dataclass
from typing import Literal

import torch

from mlx_train_perf import _compat, _native
from mlx_train_perf.core import chunked as _chunked
from mlx_train_perf.core.naive import naive_linear_ce
from mlx_train_perf.core.quant import dequantize
from mlx_train_perf.errors import LossInputError, UnsupportedHeadError
from mlx_train_perf.plan import launch as _plan

# The MI355X kernels take bf16 (bf16 MFMA, fp32 accumulation) or fp32 (fp32 MFMA) hidden states,
# as the reference kernel's element type is fp32 or bf16 (loss.py:20-24).
_KERNEL_DTYPES = (torch.bfloat16, torch.float32)
_KERNEL_ROW_TILE = 256  # token rows per workgroup tile (reported as Resolution.row_tiles)
_DEFAULT_CHUNK = 8192   # chunked-impl vocab chunk (the reference's kernel tile, loss.py:25)
_WORD_DTYPES = tuple(t for t in (torch.int32, getattr(torch, "uint32", None)) if t is not None)


@dataclass(frozen=True, slots=True, kw_only=True)
class DenseHead:
    weight: torch.Tensor      # (V, D); tied embeddings pass the same tensor
    trainable: bool = True


@dataclass(frozen=True, slots=True, kw_only=True)
class QuantizedHead:
    w_q: torch.Tensor         # int32 bit patterns of uint32 words (V, D/8)
    scales: torch.Tensor      # (V, D/64)
    biases: torch.Tensor      # (V, D/64)
    group_size: int = 64
    bits: int = 4             # frozen by definition -- no d_head path exists


HeadRef = DenseHead | QuantizedHead


def tied_head(embedding_weight: torch.Tensor, *, trainable: bool = False) -> DenseHead:
    return DenseHead(weight=embedding_weight, trainable=trainable)


@dataclass(frozen=True, slots=True, kw_only=True)
class Resolution:
    impl: Literal["kernel", "chunked", "naive"]
    row_tiles: int | None
    provisional: bool
    reason: str


def _quantized_head_d(head: QuantizedHead) -> int:
    return head.w_q.shape[-1] * (32 // head.bits)


def _require_kernel_supported(*, head: HeadRef, dtype: torch.dtype) -> None:
    """Structural gate for the kernel impl (reference loss.py:65-91): raises UnsupportedHeadError,
    naming the 'chunked' alternative, for any head/dtype combination the kernel cannot serve."""
    if dtype not in _KERNEL_DTYPES:
        raise UnsupportedHeadError(
            f"kernel impl only supports fp32/bf16 hidden dtype (got {dtype}); "
            "use impl='chunked' for other dtypes."
        )
    if isinstance(head, QuantizedHead):
        if head.bits != 4:
            raise UnsupportedHeadError(
                f"kernel impl only supports 4-bit quantized heads (got bits={head.bits}); "
                "use impl='chunked' for other bit widths."
            )
        if head.group_size != 64:
            raise UnsupportedHeadError(
                "kernel impl only supports group_size=64 quantized heads (got "
                f"group_size={head.group_size}); use impl='chunked' for other group sizes."
            )
        d = _quantized_head_d(head)
        if d % 64 != 0:
            raise UnsupportedHeadError(
                "kernel impl requires the quantized head's hidden dim to be a multiple of "
                f"64 (got d={d}); use impl='chunked'."
            )
        if head.w_q.dtype not in _WORD_DTYPES:
            raise UnsupportedHeadError(
                f"kernel impl reads w_q as 32-bit words (int32 or uint32 bit patterns); got {head.w_q.dtype}. "
                "Use impl='chunked'."
            )
        # bf16 hidden states: the kernels read scales and biases as bf16; fp32: as fp32 (either
        # stored dtype is converted, losslessly, for the fp32 kernels).
        sb_ok = (torch.bfloat16,) if dtype == torch.bfloat16 else (torch.bfloat16, torch.float32)
        for name, t in (("scales", head.scales), ("biases", head.biases)):
            if t.dtype not in sb_ok:
                raise UnsupportedHeadError(
                    f"kernel impl reads the quantized head's {name} as {'bf16' if dtype == torch.bfloat16 else 'fp32'}; "
                    f"got {t.dtype}. Use impl='chunked' (it dequantizes in the given dtype) or store them as bf16."
                )
    else:
        d = head.weight.shape[-1]
        if dtype == torch.bfloat16 and d % 8 != 0:
            raise UnsupportedHeadError(
                f"kernel impl requires the hidden dim to be a multiple of 8 (got d={d}); use impl='chunked'."
            )


def resolve_impl(*, head: HeadRef, dtype: torch.dtype, n: int, impl: str = "auto",
                 allow_unverified_mlx: bool = False) -> Resolution:
    """Resolve `auto|kernel|chunked|naive` (reference loss.py:94-123). `auto` and `kernel` resolve
    identically and never fall back; `allow_unverified_mlx` relaxes the device-architecture gate
    (the MI355X analogue of the reference's mlx version gate)."""
    if n <= 0:
        raise LossInputError(f"n must be positive (hidden's row count); got n={n}")
    if impl == "chunked":
        return Resolution(impl="chunked", row_tiles=None, provisional=False, reason="explicit impl='chunked' opt-in")
    if impl == "naive":
        return Resolution(impl="naive", row_tiles=None, provisional=False, reason="explicit impl='naive' opt-in")
    if impl not in ("auto", "kernel"):
        raise LossInputError(f"unknown impl {impl!r}; expected one of 'auto', 'kernel', 'chunked', 'naive'")
    _require_kernel_supported(head=head, dtype=dtype)
    _compat.check_device_verified(allow_unverified=allow_unverified_mlx, error=UnsupportedHeadError)
    plan = _plan.lce_plan(n=n, v=_head_v(head))
    reason = (f"kernel: {_KERNEL_ROW_TILE}-row x 256-vocab MFMA tiles, {plan.fwd_splits} vocab splits "
              f"for n={n}")
    return Resolution(impl="kernel", row_tiles=_KERNEL_ROW_TILE, provisional=False, reason=reason)


def _head_v(head: HeadRef) -> int:
    return head.weight.shape[0] if isinstance(head, DenseHead) else head.w_q.shape[0]


def _validate_inputs(*, hidden: torch.Tensor, head: HeadRef, targets: torch.Tensor, validate_targets: bool,
                     ignore_index: int) -> None:
    """Reference loss.py:126-186, plus the ignore_index exemption in the range check."""
    if hidden.dim() not in (2, 3):
        raise LossInputError(f"hidden must be 2D (N,D) or 3D (B,S,D), got shape {tuple(hidden.shape)}")
    leading = tuple(hidden.shape[:-1])
    n_total = 1
    for size in leading:
        n_total *= size
    if n_total <= 0:
        raise LossInputError(f"hidden must have at least one row, got leading dims {leading}")
    if tuple(targets.shape) != leading:
        raise LossInputError(f"targets shape {tuple(targets.shape)} must match hidden's leading dims {leading}")
    if targets.dtype.is_floating_point or targets.dtype.is_complex or targets.dtype == torch.bool:
        raise LossInputError(f"targets must be an integer dtype, got {targets.dtype}")
    d = hidden.shape[-1]
    if isinstance(head, DenseHead):
        if head.weight.dim() != 2 or head.weight.shape[-1] != d:
            raise LossInputError(f"head.weight's last dim ({head.weight.shape[-1]}) must match hidden's D ({d})")
        if hidden.dtype != head.weight.dtype:
            raise LossInputError(
                f"hidden dtype {hidden.dtype} must match dense head weight dtype {head.weight.dtype}"
            )
        v = head.weight.shape[0]
    else:
        if head.w_q.dim() != 2:
            raise LossInputError(f"w_q must be 2-D (V, D*bits/32); got shape {tuple(head.w_q.shape)}")
        head_d = _quantized_head_d(head)
        if head_d != d:
            raise LossInputError(
                f"quantized head implies D={head_d} (from w_q shape and bits), which does not match hidden's D={d}"
            )
        v = head.w_q.shape[0]
        groups = (d + head.group_size - 1) // head.group_size
        for name, t in (("scales", head.scales), ("biases", head.biases)):
            if tuple(t.shape) != (v, groups):
                raise LossInputError(
                    f"quantized head {name} must have shape (V, D/group_size)=({v}, {groups}); got {tuple(t.shape)}"
                )
    if validate_targets:
        # A host sync, skipped on the trusted training path (validate_targets=False).
        valid = targets[targets != ignore_index]
        if valid.numel():
            tmin = int(valid.min().item())
            tmax = int(valid.max().item())
            if tmin < 0 or tmax >= v:
                raise LossInputError(f"targets must satisfy 0 <= t < V={v} (or equal ignore_index); got range [{tmin}, {tmax}]")


def _reduce(nll: torch.Tensor, *, reduction: str, leading: tuple[int, ...], targets2: torch.Tensor,
            ignore_index: int) -> torch.Tensor:
    if reduction == "none":
        return nll.reshape(leading)
    if reduction == "mean":
        valid = (targets2 != ignore_index)
        return nll.sum() / valid.sum().clamp(min=1).to(nll.dtype)
    return nll.sum()


def _mask_ignored(nll: torch.Tensor, targets2: torch.Tensor, ignore_index: int) -> torch.Tensor:
    return torch.where(targets2 == ignore_index, torch.zeros_like(nll), nll)


def _naive_nll(hidden2, head, targets2, ignore_index):
    safe = torch.where(targets2 == ignore_index, torch.zeros_like(targets2), targets2)
    if isinstance(head, DenseHead):
        w = head.weight if head.trainable else head.weight.detach()
        nll = naive_linear_ce(hidden2, w, safe)
    else:
        w = dequantize(head.w_q, head.scales, head.biases, group_size=head.group_size, bits=head.bits,
                       dtype=hidden2.dtype)
        nll = naive_linear_ce(hidden2, w, safe)
    return _mask_ignored(nll, targets2, ignore_index)


def _chunked_nll(hidden2, head, targets2, ignore_index, chunk_size):
    safe = torch.where(targets2 == ignore_index, torch.zeros_like(targets2), targets2).long()
    if isinstance(head, DenseHead):
        w = head.weight if head.trainable else head.weight.detach()
        nll = _chunked.chunked_nll(hidden2, safe, chunk_size=chunk_size, weight=w)
    else:
        q = _chunked.QuantSpec(w_q=head.w_q, scales=head.scales, biases=head.biases,
                               group_size=head.group_size, bits=head.bits)
        nll = _chunked.chunked_nll(hidden2, safe, chunk_size=chunk_size, quant=q)
    return _mask_ignored(nll, targets2, ignore_index)


VJP_CALLS: dict[str, int] = {}

# Transposed copies of heads for the backward's dH product (mtp_lce_head_transpose): per device, a
# short most-recently-used list of (owner weakref, data_ptr, shape, version) -> bf16
# [D][mtp_lce_head_t_ld(V)]. The owner is the caller's weight tensor (the packed w_q of a 4-bit head,
# whose copy holds the dequantized values; kept only with MTP_LCE_TRANSPOSED_HEAD=1, since by default
# a 4-bit backward stages each vocab chunk of it in its workspace); an in-place update through it bumps its version and
# replaces its entry. A frozen head is therefore transposed once; a trainable one after every
# optimizer step. Up to MTP_LCE_HEAD_T_CACHE heads (default 2) are kept per device, so two models
# (or a model and its reference copy) on one GPU do not evict each other on every call; entries of
# heads that were freed are dropped. Guarded by a lock: trainer threads may share a device.
_HEAD_T_CACHE: dict[int, list[tuple[tuple, torch.Tensor]]] = {}
_HEAD_T_LOCK = threading.Lock()


def _head_t_capacity() -> int:
    return max(1, int(os.environ.get("MTP_LCE_HEAD_T_CACHE", "2")))


def clear_transposed_head_cache() -> None:
    """Drop the cached transposed heads (e.g. after changing a head through `.data`, which does not
    bump the tensor's version counter)."""
    with _HEAD_T_LOCK:
        _HEAD_T_CACHE.clear()


def transposed_head_cache_bytes() -> int:
    """Device bytes held by the cached transposed heads, over all devices."""
    with _HEAD_T_LOCK:
        _drop_freed_heads()
        return sum(t.numel() * t.element_size() for ents in _HEAD_T_CACHE.values() for _, t in ents)


def _drop_freed_heads() -> None:
    """Release the copies of heads that no longer exist (caller holds the lock)."""
    for ents in _HEAD_T_CACHE.values():
        ents[:] = [e for e in ents if e[0][0]() is not None]


def _transposed_head(owner: torch.Tensor | None, w, w_q, scales, biases, head_kind: int, v: int,
                     d: int) -> torch.Tensor | None:
    # MTP_LCE_TRANSPOSED_HEAD: "0" never keeps the copy, "1" keeps it for every head; by default a
    # frozen dense head keeps it, and a 4-bit or trainable head does not (its backward stages
    # chunk-wise instead).
    mode = os.environ.get("MTP_LCE_TRANSPOSED_HEAD", "auto")
    with _HEAD_T_LOCK:
        _drop_freed_heads()
    if owner is None or mode == "0" or d % 64 != 0 or (head_kind == _native.HEAD_Q4 and mode != "1"):
        return None
    dev = owner.device.index if owner.device.index is not None else torch.cuda.current_device()
    key = (owner.data_ptr(), tuple(owner.shape), owner._version)
    with _HEAD_T_LOCK:
        ents = _HEAD_T_CACHE.setdefault(dev, [])
        # drop this head's entry from before an in-place update
        ents[:] = [e for e in ents if not (e[0][0]() is owner and e[0][1:] != key)]
        for i, e in enumerate(ents):
            if e[0][0]() is owner:
                ents.append(ents.pop(i))
                return e[1]
        lib = _native.load()
        wt = torch.empty((d, lib.mtp_lce_head_t_ld(v)), dtype=torch.bfloat16, device=owner.device)
        with _native.on_device(owner):
            rc = lib.mtp_lce_head_transpose(_native.ptr(w), _native.ptr(w_q), _native.ptr(scales),
                                            _native.ptr(biases), v, d, head_kind, wt.data_ptr(),
                                            _native.stream_of(owner))
        _native.check(rc, domain="loss")
        ents.append(((weakref.ref(owner),) + key, wt))
        del ents[:-_head_t_capacity()]
        return wt


def _forward_stage_bytes(lib, n: int, d: int, v: int, head_kind: int, f32: bool) -> int:
    """Workspace of the staged 4-bit forward (MTP_HEAD_Q4_STAGED) when the loss layer runs it, else 0:
    a bf16 forward over a 4-bit head whose whole dequantization fits the workspace budget, unless
    MTP_LCE_STAGE_HEAD is "0". With less room the forward would stage runs of its vocab splits one
    launch each, every launch filling only part of the GPU: slower than dequantizing in registers."""
    if head_kind != _native.HEAD_Q4 or f32 or d % 64 or os.environ.get("MTP_LCE_STAGE_HEAD", "1") == "0":
        return 0
    ws = lib.mtp_lce_fwd_stage_workspace_bytes(n, d, v, _plan.lce_bwd_budget_bytes())
    whole = -(-lib.mtp_lce_fwd_workspace_bytes(n, d, v, _native.HEAD_Q4) // 256) * 256 + v * d * 2
    return ws if ws == whole else 0


class _KernelLCE(torch.autograd.Function):
    """Forward: mtp_lce_fwd -> (nll, lse, tgt). Backward: mtp_lce_bwd from the saved lse only; it also
    returns dL/dW when the dense head is an input that requires grad (trainable head). fp32 hidden
    states run the fp32 entry points (mtp_lce_fwd_f32 / mtp_lce_bwd_f32)."""

    @staticmethod
    def forward(ctx, hidden2, targets2, w, w_q, scales, biases, head_kind, ignore_index, bwd_chunk, owner=None):
        lib = _native.load()
        n, d = hidden2.shape
        v = w.shape[0] if head_kind == _native.HEAD_DENSE else w_q.shape[0]
        dev = hidden2.device
        f32 = hidden2.dtype == torch.float32
        nll = torch.empty(n, dtype=torch.float32, device=dev)
        lse = torch.empty(n, dtype=torch.float32, device=dev)
        tgt = torch.empty(n, dtype=torch.float32, device=dev)
        ws_fn = lib.mtp_lce_fwd_f32_workspace_bytes if f32 else lib.mtp_lce_fwd_workspace_bytes
        fwd = lib.mtp_lce_fwd_f32 if f32 else lib.mtp_lce_fwd
        fwd_kind = head_kind
        ws_bytes = _forward_stage_bytes(lib, n, d, v, head_kind, f32)
        if ws_bytes:
            # the whole 4-bit head dequantized into the workspace, then the dense product over it
            fwd_kind = _native.HEAD_Q4_STAGED
        else:
            ws_bytes = ws_fn(n, d, v, head_kind)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        with _native.on_device(hidden2):
            rc = fwd(hidden2.data_ptr(), _native.ptr(w), _native.ptr(w_q), _native.ptr(scales), _native.ptr(biases),
                     targets2.data_ptr(), n, d, v, fwd_kind, ignore_index, nll.data_ptr(), lse.data_ptr(),
                     tgt.data_ptr(), ws.data_ptr(), ws_bytes, _native.stream_of(hidden2))
        _native.check(rc, domain="loss")
        ctx.save_for_backward(hidden2, targets2, lse)
        ctx.head = (w, w_q, scales, biases, head_kind, v)
        ctx.ignore_index = ignore_index
        ctx.bwd_chunk = bwd_chunk
        ctx.owner = owner
        ctx.mark_non_differentiable(lse, tgt)
        return nll, lse, tgt

    @staticmethod
    def backward(ctx, d_nll, _d_lse, _d_tgt):
        VJP_CALLS["kernel"] = VJP_CALLS.get("kernel", 0) + 1
        lib = _native.load()
        hidden2, targets2, lse = ctx.saved_tensors
        w, w_q, scales, biases, head_kind, v = ctx.head
        n, d = hidden2.shape
        d_w = torch.empty_like(w) if (w is not None and ctx.needs_input_grad[2]) else None
        if hidden2.dtype == torch.float32:
            return _f32_backward(lib, ctx, hidden2, targets2, lse, d_nll, d_w)
        vpad = (v + 255) // 256 * 256
        # A trainable head changes at every optimizer step, so a cached copy would be rebuilt every
        # step and held between them: by default its backward stages its chunks instead.
        w_t = (None if d_w is not None and os.environ.get("MTP_LCE_TRANSPOSED_HEAD", "auto") != "1"
               else _transposed_head(ctx.owner, w, w_q, scales, biases, head_kind, v, d))
        # A head without the cached transposed copy stages each vocab chunk of it, transposed (a 4-bit
        # head dequantized), in the workspace (MTP_LCE_STAGE_HEAD=0: the dH product reads W through
        # LDS transpose reads, or dequantizes the packed words in registers, with no staging buffer).
        staged = w_t is None and d % 64 == 0 and os.environ.get("MTP_LCE_STAGE_HEAD", "1") != "0"
        if staged:
            head_kind = _native.HEAD_Q4_STAGED if head_kind == _native.HEAD_Q4 else _native.HEAD_DENSE_STAGED
        if ctx.bwd_chunk:   # an explicit vocab chunk: all rows in one block
            chunk, rows = min(max(256, (ctx.bwd_chunk + 255) // 256 * 256), vpad), n
        elif staged:   # every row block would stage every chunk again
            chunk, rows = lib.mtp_lce_bwd_stage_chunk(n, d, v, head_kind, _plan.lce_bwd_budget_bytes()), n
        else:
            # Row blocks reuse one gradient buffer (a trainable head's dL/dW needs every row at once).
            budget = _plan.lce_bwd_budget_bytes()
            rows = n if d_w is not None else lib.mtp_lce_bwd_row_block(n, d, v, budget)
            chunk = vpad if rows < n else lib.mtp_lce_bwd_chunk(n, d, v, budget)
        ws_bytes = lib.mtp_lce_bwd_workspace_bytes(n, d, v, head_kind, chunk, rows)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=hidden2.device)
        d_hidden = torch.empty_like(hidden2)
        ct = d_nll.to(torch.float32).contiguous()
        with _native.on_device(hidden2):
            rc = lib.mtp_lce_bwd(hidden2.data_ptr(), _native.ptr(w), _native.ptr(w_t), _native.ptr(w_q),
                                 _native.ptr(scales), _native.ptr(biases), targets2.data_ptr(), n, d, v, head_kind,
                                 ctx.ignore_index, lse.data_ptr(), ct.data_ptr(), d_hidden.data_ptr(),
                                 _native.ptr(d_w), chunk, rows, ws.data_ptr(), ws_bytes, _native.stream_of(hidden2))
        _native.check(rc, domain="loss")
        return d_hidden, None, d_w, None, None, None, None, None, None, None


def _f32_backward(lib, ctx, hidden2, targets2, lse, d_nll, d_w):
    """mtp_lce_bwd_f32: fp32 gradient tiles per vocab chunk (a multiple of 128 planned from the
    workspace budget, or the caller's chunk), dH (and a trainable head's dW) in fp32."""
    w, w_q, scales, biases, head_kind, v = ctx.head
    n, d = hidden2.shape
    vpad = (v + 127) // 128 * 128
    if ctx.bwd_chunk:
        chunk = min(max(128, (ctx.bwd_chunk + 127) // 128 * 128), vpad)
    else:
        chunk = lib.mtp_lce_bwd_f32_chunk(n, d, v, _plan.lce_bwd_budget_bytes())
    ws_bytes = lib.mtp_lce_bwd_f32_workspace_bytes(n, d, v, chunk)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=hidden2.device)
    d_hidden = torch.empty_like(hidden2)
    ct = d_nll.to(torch.float32).contiguous()
    with _native.on_device(hidden2):
        rc = lib.mtp_lce_bwd_f32(hidden2.data_ptr(), _native.ptr(w), _native.ptr(w_q), _native.ptr(scales),
                                 _native.ptr(biases), targets2.data_ptr(), n, d, v, head_kind, ctx.ignore_index,
                                 lse.data_ptr(), ct.data_ptr(), d_hidden.data_ptr(), _native.ptr(d_w), chunk,
                                 ws.data_ptr(), ws_bytes, _native.stream_of(hidden2))
    _native.check(rc, domain="loss")
    return d_hidden, None, d_w, None, None, None, None, None, None, None


def _require_same_device(hidden2: torch.Tensor, head: HeadRef, targets2: torch.Tensor) -> None:
    """Every tensor the kernels read must live on hidden's GPU: a host or other-device pointer
    handed to a launch would fault the GPU instead of raising."""
    _compat.require_gpu_tensor(hidden2, error=UnsupportedHeadError)
    parts = [("targets", targets2)]
    if isinstance(head, DenseHead):
        parts.append(("head.weight", head.weight))
    else:
        parts += [("head.w_q", head.w_q), ("head.scales", head.scales), ("head.biases", head.biases)]
    for name, t in parts:
        if t.device != hidden2.device:
            raise LossInputError(f"{name} is on {t.device} but hidden is on {hidden2.device}; the kernel impl "
                                 "needs every input on the same GPU")


def kernel_forward_parts(hidden2: torch.Tensor, head: HeadRef, targets2: torch.Tensor, *, ignore_index: int = -100,
                         bwd_chunk: int | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(nll, lse, tgt) from the kernel impl, differentiable in hidden2 through `nll` (test/bench seam)."""
    _require_same_device(hidden2, head, targets2)
    h = hidden2.contiguous()
    t = targets2.to(torch.int64).contiguous()
    if isinstance(head, DenseHead):
        w = head.weight if head.trainable else head.weight.detach()
        if not w.is_contiguous():
            raise UnsupportedHeadError("kernel impl needs a contiguous (V, D) head weight")
        return _KernelLCE.apply(h, t, w, None, None, None, _native.HEAD_DENSE, int(ignore_index), int(bwd_chunk or 0),
                                head.weight)
    sb = torch.float32 if h.dtype == torch.float32 else torch.bfloat16   # the fp32 kernels read fp32 scales
    args = (None, head.w_q.contiguous(), head.scales.to(sb).contiguous(), head.biases.to(sb).contiguous(),
            _native.HEAD_Q4)
    return _KernelLCE.apply(h, t, *args, int(ignore_index), int(bwd_chunk or 0), head.w_q)


def linear_cross_entropy(
    hidden: torch.Tensor,
    head: HeadRef,
    targets: torch.Tensor,
    *,
    impl: Literal["auto", "kernel", "chunked", "naive"] = "auto",
    chunk_size: int | None = None,
    reduction: Literal["none", "mean", "sum"] = "mean",
    allow_unverified_mlx: bool = False,
    validate_targets: bool = True,
    ignore_index: int = -100,
) -> torch.Tensor:
    """Fused linear cross-entropy of `hidden @ head.T` against `targets` (reference loss.py:358-392).

    `chunk_size`: vocab chunk of the chunked impl; for the kernel impl, the backward's vocab chunk
    (rounded up to a multiple of 256; default: planned from the workspace budget)."""
    if reduction not in ("none", "mean", "sum"):
        raise LossInputError(f"unknown reduction {reduction!r}; expected 'none', 'mean', or 'sum'")
    _validate_inputs(hidden=hidden, head=head, targets=targets, validate_targets=validate_targets,
                     ignore_index=ignore_index)
    leading = tuple(hidden.shape[:-1])
    hidden2 = hidden.reshape(-1, hidden.shape[-1])
    targets2 = targets.reshape(-1)
    n = hidden2.shape[0]
    res = resolve_impl(head=head, dtype=hidden2.dtype, n=n, impl=impl, allow_unverified_mlx=allow_unverified_mlx)
    if res.impl == "naive":
        nll = _naive_nll(hidden2, head, targets2, ignore_index)
    elif res.impl == "chunked":
        nll = _chunked_nll(hidden2, head, targets2, ignore_index, _DEFAULT_CHUNK if chunk_size is None else chunk_size)
    else:
        nll, _, _ = kernel_forward_parts(hidden2, head, targets2, ignore_index=ignore_index, bwd_chunk=chunk_size)
    return _reduce(nll, reduction=reduction, leading=leading, targets2=targets2, ignore_index=ignore_index)
