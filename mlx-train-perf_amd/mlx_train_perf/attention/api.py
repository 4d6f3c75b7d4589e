"""`flash_attention` public API (mirror of src/mlx_train_perf/attention/api.py on torch tensors).

Residual contract (api.py:1-18): the autograd Function returns (O, L); L is a real output, marked
non-differentiable, and only O reaches the caller. The backward reads q, k, v and the saved O, L.

`impl="auto"`/`"kernel"`: the HIP kernels of libmtp_hip.so (bf16 on bf16 MFMA, fp32 on fp32 MFMA
with fp32 outputs and gradients; head_dim in {64, 96, 128}; causal with optional packed segments,
or non-causal -- an extension: the reference kernel refuses causal=False, api.py:109-113). `impl="reference"`: the materialized oracle with the hand-written
FlashAttention backward over full tensors -- an explicit opt-in, O(N^2) memory, small N only.
No silent fallback: unsupported configs raise the reference's typed errors.
"""
from __future__ import annotations

import weakref
from typing import Literal

import torch

from mlx_train_perf import _compat, _native
from mlx_train_perf.attention.reference import flash_attention_reference, kv_head_for
from mlx_train_perf.attention.segments import PackedMask, layout_violation, segment_allowed
from mlx_train_perf.errors import AttentionInputError, UnsupportedAttentionError

_KERNEL_DTYPES = (torch.bfloat16, torch.float32)   # the reference kernel's T (api.py:41-43)
_KERNEL_HEAD_DIMS = (64, 96, 128)

VJP_CALLS: dict[str, int] = {}


def _validate_shapes(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """api.py:52-72."""
    for name, arr in (("q", q), ("k", k), ("v", v)):
        if arr.dim() != 4:
            raise AttentionInputError(f"{name} must be 4-D (B, H, N, D); got shape {tuple(arr.shape)}")
    b_q, hq, n_q, d_q = q.shape
    b_k, hkv, n_k, d_k = k.shape
    b_v, hv, n_v, d_v = v.shape
    if b_q < 1:
        raise AttentionInputError(f"batch must be >= 1; got {b_q}")
    if not (b_q == b_k == b_v):
        raise AttentionInputError(f"batch mismatch: q={b_q}, k={b_k}, v={b_v}")
    if hkv != hv:
        raise AttentionInputError(f"k/v head-count mismatch: k has {hkv} heads, v has {hv}")
    if hq % hkv != 0:
        raise AttentionInputError(f"Hq={hq} must be a multiple of Hkv={hkv} for GQA grouping")
    if not (n_q == n_k == n_v):
        raise AttentionInputError(f"sequence length mismatch: q={n_q}, k={n_k}, v={n_v}")
    if not (d_q == d_k == d_v):
        raise AttentionInputError(f"head_dim mismatch: q={d_q}, k={d_k}, v={d_v}")
    if not (q.device == k.device == v.device):
        raise AttentionInputError(f"q, k, v must be on one device; got {q.device}, {k.device}, {v.device}")


# Segment tensors whose layout passed `layout_violation`: weak references to the two tensors and their
# version counters. A model calls flash_attention once per layer with the same mask, so the check
# (one device pass and a host sync) runs once per mask rather than once per layer; an in-place edit
# bumps a version and a new tensor is a new object, so either is checked again.
_CHECKED_LAYOUTS: dict[int, tuple] = {}


def _layout_seen(segments: PackedMask) -> bool:
    ent = _CHECKED_LAYOUTS.get(id(segments.seg_id))
    return (ent is not None and ent[0]() is segments.seg_id and ent[1]() is segments.seg_start
            and ent[2] == (segments.seg_id._version, segments.seg_start._version))


def _validate_segments(q: torch.Tensor, segments: PackedMask, *, check_layout: bool = False) -> None:
    b, _, n, _ = q.shape
    for name, t in (("seg_id", segments.seg_id), ("seg_start", segments.seg_start)):
        if tuple(t.shape) != (b, n):
            raise AttentionInputError(f"segments.{name} must have shape (B, N)=({b}, {n}); got {tuple(t.shape)}")
        if t.dtype.is_floating_point or t.dtype == torch.bool or t.dtype.is_complex:
            raise AttentionInputError(f"segments.{name} must be an integer tensor; got {t.dtype}")
    if check_layout and not _layout_seen(segments):
        problem = layout_violation(segments.seg_id, segments.seg_start)
        if problem is not None:
            raise AttentionInputError(f"segments violate the packed-row layout contract: {problem}")
        if len(_CHECKED_LAYOUTS) > 64:
            _CHECKED_LAYOUTS.clear()
        sid, sst = segments.seg_id, segments.seg_start
        _CHECKED_LAYOUTS[id(sid)] = (weakref.ref(sid), weakref.ref(sst), (sid._version, sst._version))


def resolve_attention_impl(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, impl: str, causal: bool = True,
                           segments: PackedMask | None = None, validate_segments: bool = False) -> str:
    """api.py:75-123: "reference" is always allowed; "auto"/"kernel" run the kernel-support gate."""
    _validate_shapes(q, k, v)
    if segments is not None:
        _validate_segments(q, segments, check_layout=validate_segments)
        if not causal:
            raise UnsupportedAttentionError(
                "segments (packed attention) require causal=True (got causal=False); "
                "packing composes on top of the causal triangle."
            )
    if impl == "reference":
        return "reference"
    if impl not in ("auto", "kernel"):
        raise AttentionInputError(f"unknown impl {impl!r}; expected one of 'auto', 'kernel', 'reference'")
    if q.dtype not in _KERNEL_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise UnsupportedAttentionError(
            f"kernel impl only supports fp32/bf16 (got {q.dtype}/{k.dtype}/{v.dtype}); use impl='reference'."
        )
    head_dim = q.shape[-1]
    if head_dim not in _KERNEL_HEAD_DIMS:
        raise UnsupportedAttentionError(
            f"kernel impl only supports head_dim in {_KERNEL_HEAD_DIMS} (got {head_dim}); use impl='reference'."
        )
    _compat.check_device_verified(allow_unverified=False, error=UnsupportedAttentionError)
    _compat.require_gpu_tensor(q, error=UnsupportedAttentionError)
    return "kernel"


def _bwd_D(d_o: torch.Tensor, o: torch.Tensor) -> torch.Tensor:  # noqa: N802 -- the paper's name
    """D_i = sum_d dO_i,d O_i,d in fp32 (api.py:126-129)."""
    return (d_o.to(torch.float32) * o.to(torch.float32)).sum(dim=-1)


def _kv_gather(x: torch.Tensor, *, hq: int, hkv: int) -> torch.Tensor:
    group = hq // hkv
    idx = torch.tensor([kv_head_for(h, group) for h in range(hq)], device=x.device)
    return x.index_select(1, idx)


def _flash_attention_backward(q, k, v, o, lse, d_o, *, scale, causal, segments=None):
    """Hand-written FlashAttention backward over full tensors, fp32 (api.py:140-194)."""
    b, hq, n, dd = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    q32 = q.to(torch.float32)
    k_g = _kv_gather(k, hq=hq, hkv=hkv).to(torch.float32)
    v_g = _kv_gather(v, hq=hq, hkv=hkv).to(torch.float32)
    d = _bwd_D(d_o, o)
    do32 = d_o.to(torch.float32)
    s = (q32 @ k_g.transpose(-1, -2).contiguous()) * scale
    if segments is not None:
        s = s.masked_fill(~segment_allowed(segments.seg_id), float("-inf"))
    if causal:
        s = s.masked_fill(torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1), float("-inf"))
    p = torch.exp(s - lse.to(torch.float32)[..., None])
    d_p = do32 @ v_g.transpose(-1, -2).contiguous()
    d_s = p * (d_p - d[..., None])
    d_q = scale * (d_s @ k_g)
    d_v = (p.transpose(-1, -2).contiguous() @ do32).reshape(b, hkv, group, n, dd).sum(2)
    d_k = (scale * (d_s.transpose(-1, -2).contiguous() @ q32)).reshape(b, hkv, group, n, dd).sum(2)
    return d_q.to(q.dtype), d_k.to(k.dtype), d_v.to(v.dtype)


class _ReferenceAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, seg_id, seg_start, scale, causal):
        segments = None if seg_id is None else PackedMask(seg_id=seg_id, seg_start=seg_start)
        o, lse = flash_attention_reference(q, k, v, scale=scale, causal=causal, segments=segments)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.segments = segments
        ctx.scale, ctx.causal = scale, causal
        ctx.mark_non_differentiable(lse)
        return o, lse

    @staticmethod
    def backward(ctx, d_o, _d_l):
        VJP_CALLS["flash_attention"] = VJP_CALLS.get("flash_attention", 0) + 1
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _flash_attention_backward(q, k, v, o, lse, d_o, scale=ctx.scale, causal=ctx.causal,
                                               segments=ctx.segments)
        return dq, dk, dv, None, None, None, None


def _seg_args(q, seg_id, seg_start):
    if seg_id is None:
        return None, None
    return seg_id.to(device=q.device, dtype=torch.int32).contiguous(), \
        seg_start.to(device=q.device, dtype=torch.int32).contiguous()


def kernel_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float,
                   seg_id: torch.Tensor | None = None, seg_start: torch.Tensor | None = None, causal: bool = True):
    """(O, L) from mtp_attn_fwd; q/k/v contiguous bf16 on the GPU. causal=False: every key visible."""
    lib = _native.load()
    b, hq, n, dh = q.shape
    hkv = k.shape[1]
    o = torch.empty_like(q)
    lse = torch.empty((b, hq, n), dtype=torch.float32, device=q.device)
    fwd = lib.mtp_attn_fwd_f32 if q.dtype == torch.float32 else lib.mtp_attn_fwd
    with _native.on_device(q):
        rc = fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), b, hq, hkv, n, dh, float(scale), int(causal),
                 _native.ptr(seg_id), _native.ptr(seg_start), o.data_ptr(), lse.data_ptr(), _native.stream_of(q))
    _native.check(rc, domain="attention")
    return o, lse


def kernel_backward(q, k, v, o, lse, d_o, *, scale: float, seg_id=None, seg_start=None, causal: bool = True):
    """(dQ, dK, dV) from mtp_attn_bwd (mtp_attn_bwd_f32 for fp32 inputs)."""
    lib = _native.load()
    b, hq, n, dh = q.shape
    hkv = k.shape[1]
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    f32 = q.dtype == torch.float32
    ws_bytes = (lib.mtp_attn_bwd_f32_workspace_bytes if f32 else lib.mtp_attn_bwd_workspace_bytes)(b, hq, hkv, n, dh)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    bwd = lib.mtp_attn_bwd_f32 if f32 else lib.mtp_attn_bwd
    with _native.on_device(q):
        rc = bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), d_o.data_ptr(), b, hq, hkv,
                 n, dh, float(scale), int(causal), _native.ptr(seg_id), _native.ptr(seg_start), dq.data_ptr(),
                 dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, _native.stream_of(q))
    _native.check(rc, domain="attention")
    return dq, dk, dv


class _KernelAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, seg_id, seg_start, scale, causal):
        o, lse = kernel_forward(q, k, v, scale=scale, seg_id=seg_id, seg_start=seg_start, causal=causal)
        ctx.save_for_backward(q, k, v, o, lse, seg_id, seg_start)
        ctx.scale, ctx.causal = scale, causal
        ctx.mark_non_differentiable(lse)
        return o, lse

    @staticmethod
    def backward(ctx, d_o, _d_l):
        VJP_CALLS["flash_attention"] = VJP_CALLS.get("flash_attention", 0) + 1
        VJP_CALLS["flash_attention_kernel_bwd"] = VJP_CALLS.get("flash_attention_kernel_bwd", 0) + 1
        q, k, v, o, lse, seg_id, seg_start = ctx.saved_tensors
        dq, dk, dv = kernel_backward(q, k, v, o, lse, d_o.contiguous(), scale=ctx.scale, seg_id=seg_id,
                                     seg_start=seg_start, causal=ctx.causal)
        return dq, dk, dv, None, None, None, None


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, causal: bool = True,
                    impl: Literal["auto", "kernel", "reference"] = "auto",
                    segments: PackedMask | None = None, validate_segments: bool = True) -> torch.Tensor:
    """softmax(scale * Q K^T + mask) V with GQA (api.py:281-439). Only O is returned; L stays internal.

    `segments` (requires causal=True) switches on packed block-diagonal-causal attention; the
    segment tensors are passed to the kernels per call (never captured), so every step masks with
    its own layout. `validate_segments` checks the layout contract of `PackedMask` (seg_id from 0 in
    steps of 0 or 1, seg_start the first position of each segment) and raises AttentionInputError
    on a violation; the check costs one host sync per distinct mask (a model's layers share it).
    Pass False on a trusted path, like the loss's `validate_targets`."""
    resolved = resolve_attention_impl(q, k, v, impl=impl, causal=causal, segments=segments,
                                      validate_segments=validate_segments)
    seg_id, seg_start = (None, None) if segments is None else _seg_args(q, segments.seg_id, segments.seg_start)
    if resolved == "kernel":
        o, _ = _KernelAttention.apply(q.contiguous(), k.contiguous(), v.contiguous(), seg_id, seg_start, float(scale),
                                      bool(causal))
        return o
    o, _ = _ReferenceAttention.apply(q, k, v, seg_id, seg_start, float(scale), causal)
    return o
