"""Memory planner for the hot path, sized for one MI355X (288 GB HBM3E).

The reference fits empirical coefficients for a 32 GB unified-memory Mac (plan/estimate.py,
calibration_data.json). Its hot-path terms are analytic and are kept here, re-derived for this
build's kernels and workspaces:
- loss layer (`_loss_bytes`, plan/estimate.py:252-271): kernel forward = the three fp32 outputs
  plus the vocab-split partials; the backward adds the bf16 gradient chunk and (multi-chunk) the
  fp32 dH accumulator; chunked = fp32 logits chunk x 3; naive = the full (N, V) fp32 logits plus
  softmax intermediates; a trainable head adds its dL/dW (the reference's `d_w` term) and takes
  every row in one backward block; the kernel backward also keeps a transposed copy of the head, or,
  without it (a 4-bit head by default), stages one transposed vocab chunk of the head in its
  workspace;
- flash-attention saved state (`_flash_saved_state_bytes`, plan/estimate.py:210-220): O in the
  compute dtype plus the fp32 L per layer, and the backward's fp32 D vector.
Whole-model terms (weights, optimizer, activations) are caller-supplied because they depend on the
model, not on this path.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

from mlx_train_perf.errors import DoesNotFitError, PlanInputError
from mlx_train_perf.plan import launch as _launch

HBM_BYTES_MI355X = 288 * 10**9
_DTYPE_BYTES = {"bf16": 2, "bfloat16": 2, "fp16": 2, "float16": 2, "fp32": 4, "float32": 4}


def dtype_bytes(dtype: str) -> int:
    try:
        return _DTYPE_BYTES[dtype]
    except KeyError:
        raise PlanInputError(f"unknown dtype {dtype!r}; expected one of {sorted(_DTYPE_BYTES)}") from None


@dataclass(frozen=True)
class LossBytes:
    forward_peak: int
    backward_workspace: int
    # The backward's cached transposed head (kernel impl; resident from the first backward for as
    # long as the head lives, so it adds to the forward of later steps too).
    transposed_head: int = 0
    # dL/dW of a trainable head, in the head's dtype (the reference's `d_w` term,
    # plan/estimate.py:245-271).
    head_grad: int = 0

    @property
    def backward_peak(self) -> int:
        return self.backward_workspace + self.head_grad

    @property
    def peak(self) -> int:
        """The loss layer's peak over a training step, beyond its inputs and dH."""
        return self.transposed_head + max(self.forward_peak, self.backward_peak)


def transposed_head_bytes(*, d: int, v: int, enabled: bool | None = None, quantized: bool = False,
                          trainable: bool = False) -> int:
    """One cached transposed head, bf16 [d][round_up(v, 256) + 64] (mtp_lce_head_t_ld), which the
    kernel backward keeps per head when d % 64 == 0: by default for a frozen dense head, not for a
    4-bit or a trainable one (`MTP_LCE_TRANSPOSED_HEAD` "0": for none, "1": for all)."""
    if enabled is None:
        mode = os.environ.get("MTP_LCE_TRANSPOSED_HEAD", "auto")
        enabled = mode == "1" or (mode != "0" and not quantized and not trainable)
    if not enabled or d % 64:
        return 0
    return d * (-(-v // _launch.TILE) * _launch.TILE + _launch.G_PITCH_PAD) * 2


def loss_bytes(*, n: int, d: int, v: int, impl: str = "kernel", dtype: str = "bf16", chunk: int | None = None,
               bwd_budget: int | None = None, trainable: bool = False,
               transposed_head: bool | None = None, quantized: bool = False) -> LossBytes:
    """Loss-layer memory beyond its inputs: forward marginal peak, backward workspace, and (kernel
    impl) the cached transposed head; a trainable head adds its dL/dW and, on the kernel impl, takes
    every row in one backward block. A head without the cached copy (a 4-bit head by default)
    stages each vocab chunk of it in the backward's workspace instead (unless `MTP_LCE_STAGE_HEAD`
    is "0"), over all rows; a 4-bit head's bf16 forward stages the whole head, dequantized, in its
    workspace when that fits the same budget. The backward's returned dH (n*d*dtype) is the
    caller's gradient, not counted here."""
    if n < 1 or d < 1 or v < 1:
        raise PlanInputError("n, d, v must be >= 1")
    eb = dtype_bytes(dtype)
    head_grad = v * d * eb if trainable else 0
    if impl == "kernel":
        head_t = transposed_head_bytes(d=d, v=v, enabled=transposed_head, quantized=quantized, trainable=trainable)
        staged = head_t == 0 and d % 64 == 0 and os.environ.get("MTP_LCE_STAGE_HEAD", "1") != "0"
        budget = bwd_budget or _launch.lce_bwd_budget_bytes()
        if (quantized and eb == 2 and os.environ.get("MTP_LCE_STAGE_HEAD", "1") != "0"
                and _launch.lce_fwd_stages_whole_head(n, d, v, budget)):
            fwd = 3 * n * 4 + _launch.lce_fwd_stage_workspace_bytes(n, d, v, budget)
        else:
            fwd = 3 * n * 4 + _launch.lce_fwd_workspace_bytes(n, v)
        if chunk:
            bwd = _launch.lce_bwd_workspace_bytes(n, d, v, chunk, staged=staged, quantized=quantized) + n * 4
        else:
            p = _launch.lce_plan(n=n, v=v, d=d, budget=budget, trainable=trainable, staged=staged,
                                 quantized=quantized)
            bwd = p.bwd_workspace_bytes + n * 4
        return LossBytes(forward_peak=fwd, backward_workspace=bwd, head_grad=head_grad, transposed_head=head_t)
    elif impl == "chunked":
        c = chunk or 8192
        fwd = 3 * n * min(c, v) * 4 + 2 * n * 4
        bwd = 3 * n * min(c, v) * 4 + n * d * 4 + n * min(c, v) * eb
    elif impl == "naive":
        fwd = 2 * n * v * 4 + n * v * eb
        bwd = 2 * n * v * 4
    else:
        raise PlanInputError(f"unknown impl {impl!r}; expected 'naive', 'chunked', or 'kernel'")
    return LossBytes(forward_peak=fwd, backward_workspace=bwd, head_grad=head_grad)


def flash_saved_state_bytes(*, batch: int, seq_len: int, heads: int, head_dim: int, dtype: str = "bf16") -> int:
    """Per attention layer: O (batch*heads*seq*head_dim, compute dtype) + L (batch*heads*seq fp32)."""
    return batch * heads * seq_len * head_dim * dtype_bytes(dtype) + batch * heads * seq_len * 4


def stock_attention_bytes(*, batch: int, seq_len: int, heads: int) -> int:
    """One layer's materialized fp32 (S, S) scores + probabilities, what the flash path removes."""
    return 2 * batch * heads * seq_len * seq_len * 4


@dataclass
class Plan:
    components: dict[str, int] = field(default_factory=dict)

    @property
    def total(self) -> int:
        return sum(self.components.values())


def estimate_peak(*, n_layers: int, batch: int, seq_len: int, hidden: int, vocab: int, heads: int, kv_heads: int,
                  head_dim: int, dtype: str = "bf16", attention: str = "flash", loss_impl: str = "kernel",
                  weights_bytes: int = 0, optimizer_bytes: int = 0, activation_bytes: int = 0,
                  trainable_head: bool = False, quantized_head: bool = False) -> Plan:
    """Predicted peak bytes of a training step: hot-path terms computed here, model terms supplied.
    `trainable_head` (full fine-tuning; the reference's `lora_rank == 0`, plan/estimate.py:245-250)
    adds the head's dL/dW and plans the loss backward with every row in one block;
    `quantized_head` (QLoRA) plans the 4-bit head's backward."""
    if heads % kv_heads:
        raise PlanInputError(f"heads={heads} must be a multiple of kv_heads={kv_heads}")
    n = batch * seq_len
    lb = loss_bytes(n=n, d=hidden, v=vocab, impl=loss_impl, dtype=dtype, trainable=trainable_head,
                    quantized=quantized_head)
    if attention == "flash":
        attn = n_layers * flash_saved_state_bytes(batch=batch, seq_len=seq_len, heads=heads, head_dim=head_dim,
                                                  dtype=dtype) + batch * heads * seq_len * 4
    elif attention == "stock":
        attn = stock_attention_bytes(batch=batch, seq_len=seq_len, heads=heads)
    else:
        raise PlanInputError(f"unknown attention {attention!r}; expected 'stock' or 'flash'")
    return Plan(components={
        "weights": weights_bytes, "optimizer": optimizer_bytes, "activations": activation_bytes,
        "attention": attn, "loss": lb.peak,
    })


def plan_fit(plan: Plan, *, budget_bytes: int | None = None, headroom: float = 0.05) -> int:
    """Return the planned peak, raising DoesNotFitError above (1 - headroom) * budget (default:
    the free memory of the current GPU when one is visible, else 288 GB)."""
    if budget_bytes is None:
        budget_bytes = HBM_BYTES_MI355X
        try:
            import torch  # noqa: PLC0415

            if torch.cuda.is_available():
                budget_bytes = torch.cuda.mem_get_info()[0]
        except Exception:  # noqa: BLE001 -- a planner must work without a GPU
            pass
    limit = int(budget_bytes * (1 - headroom))
    if plan.total > limit:
        raise DoesNotFitError(f"predicted peak {plan.total / 1e9:.2f} GB exceeds {limit / 1e9:.2f} GB "
                              f"({', '.join(f'{k}={v / 1e9:.2f}' for k, v in plan.components.items())})")
    return plan.total
