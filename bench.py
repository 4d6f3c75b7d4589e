"""Bench harness: fused linear cross-entropy fwd+bwd on one MI355X (config 2), with the
flash-attention (configs 4, 5), QLoRA (config 3), a trainable-head step (dL/dW), size ladders and
CPU baselines reported beside it.

The five workloads are the reference's published configurations, numbered as it numbers them:
  1  LCE, N=1024, D=512, V=32000, fp32, 10% ignore_index (the CPU-runnable case);
  2  LCE, N=8192 (batch 1 x seq 8192), D=4096, V=151936, bf16 dense frozen head (the headline);
  3  config 2 with the head quantized to 4 bits (affine, groups of 64, bf16 scales and biases);
  4  causal GQA flash attention, B=1, Hq=32, Hkv=8, S=8192, head_dim 128, bf16;
  5  config 4's heads over a packed row of S=16384 tokens, document lengths uniform in
     [64, 2048] from seed 0 (the last one truncated).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extras] [--parts ...]

One step = one LCE forward + backward (dL/dH, frozen head) at N=8192 (batch 1 x seq 8192), D=4096,
V=151936, bf16, synthetic seeded inputs resident in HBM before the timed region. Prints ONE JSON line.

Per the reference's bench discipline (src/mlx_train_perf/bench/worker.py:93-142,
scripts/bench_attention_op.py:225-296, scripts/bench_loss_layer.py:44-142): seeded inputs, warm-up
outside the window, timed window bracketed by device synchronization, medians of repeated runs for
the ladders and the CPU baselines; marginal peak memory measured the worker's way
(max_memory_allocated - allocated_before after a reset).

Profiling modes (their output is what profiles/ holds):
    python bench.py --pmc-workload                      # the program rocprofv3 --pmc passes profile
    python bench.py --pmc-summary CMD DIR [DIR ...]     # counters of those passes -> markdown
    python bench.py --trace-summary CSV TITLE CMD [STATS] # rocprofv3 --kernel-trace (--stats) csv -> markdown
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "mlx-train-perf_amd"))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (no sparsity)
PEAK_FP32_TFLOPS = 157.3    # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0

N, D, V = 8192, 4096, 151936
IGNORE = -100
ATT_B, ATT_HQ, ATT_HKV, ATT_DH = 1, 32, 8, 128


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def lce_inputs_gpu(n, d, v, seed=0, ignore_frac=0.05):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    h = torch.randn(n, d, generator=g, device="cuda")
    h = (h / torch.sqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    w = (torch.randn(v, d, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device="cuda")
    k = int(round(ignore_frac * n))
    t[torch.randperm(n, generator=g, device="cuda")[:k]] = IGNORE
    return h, w, t


def packed_lengths(total: int, lo: int = 64, hi: int = 2048, seed: int = 0) -> list[int]:
    """Config 5: document lengths uniform in [lo, hi] from `seed` until `total` is filled."""
    import random

    rng = random.Random(seed)
    lens, used = [], 0
    while used < total:
        n = min(rng.randint(lo, hi), total - used)
        lens.append(n)
        used += n
    return lens


def time_region(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def event_ms(fn, reps, warmup=2):
    """Per-call durations (ms) of `fn` with HIP events on torch's current stream, the stream every
    launch here is issued on."""
    import torch

    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    for a, b in ev:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def marginal_peak_bytes(fn):
    """max_memory_allocated - allocated_before around fn (bench/worker.py:117-132 semantics)."""
    import torch

    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - before
    return peak, out


def mfma_ceiling_tflops():
    import torch

    from mlx_train_perf import _native

    lib = _native.load()
    blocks, iters = 1024, 20000
    out = torch.zeros(blocks, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    lib.mtp_bench_mfma_ceiling(blocks, 100, out.data_ptr(), s)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    lib.mtp_bench_mfma_ceiling(blocks, iters, out.data_ptr(), s)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    flops = blocks * 4 * 4 * iters * 32768.0
    return flops / (ms * 1e-3) / 1e12


# ------------------------------------------------------------------------------------------------
# LCE (configs 2, 3)
# ------------------------------------------------------------------------------------------------
def _lce_head(w, head_kind):
    from mlx_train_perf.core.loss import DenseHead, QuantizedHead
    from mlx_train_perf.core.quant import quantize

    if head_kind == "dense":
        return DenseHead(weight=w, trainable=False)
    wq, sc, bi = quantize(w)
    return QuantizedHead(w_q=wq, scales=sc, biases=bi)


def _fwd_launcher(h, head, t, head_kind):
    """A closure issuing one mtp_lce_fwd (the roofline kernel + its finalize) through the C-ABI."""
    import torch

    from mlx_train_perf import _native
    from mlx_train_perf.plan import launch as plan

    lib = _native.load()
    n_, d_ = h.shape
    v_ = head.weight.shape[0] if head_kind == "dense" else head.w_q.shape[0]
    outs = [torch.empty(n_, dtype=torch.float32, device="cuda") for _ in range(3)]
    kind = _native.HEAD_DENSE if head_kind == "dense" else _native.HEAD_Q4
    ws_b = lib.mtp_lce_fwd_workspace_bytes(n_, d_, v_, kind)
    if (kind == _native.HEAD_Q4 and os.environ.get("MTP_LCE_STAGE_HEAD", "1") != "0"
            and plan.lce_fwd_stages_whole_head(n_, d_, v_, plan.lce_bwd_budget_bytes())):
        # the loss layer's default 4-bit forward: the head dequantized into the workspace
        kind = _native.HEAD_Q4_STAGED
        ws_b = lib.mtp_lce_fwd_stage_workspace_bytes(n_, d_, v_, plan.lce_bwd_budget_bytes())
    ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
    args = ((head.weight.data_ptr(), None, None, None) if head_kind == "dense" else
            (None, head.w_q.data_ptr(), head.scales.data_ptr(), head.biases.data_ptr()))

    def launch():
        rc = lib.mtp_lce_fwd(h.data_ptr(), *args, t.data_ptr(), n_, d_, v_, kind, IGNORE, outs[0].data_ptr(),
                             outs[1].data_ptr(), outs[2].data_ptr(), ws.data_ptr(), ws_b,
                             torch.cuda.current_stream().cuda_stream)
        _native.check(rc, domain="loss")

    return launch


def bench_lce(steps, warmup, head_kind="dense"):
    """LCE fwd+bwd step timing, per-launch event timing of the forward, per-phase times, memory."""
    import torch

    from mlx_train_perf.core import loss as L
    from mlx_train_perf.plan import launch as plan

    h, w, t = lce_inputs_gpu(N, D, V)
    head = _lce_head(w, head_kind)
    if head_kind != "dense":
        del w
    hd = h.detach().requires_grad_(True)
    valid = (t != IGNORE)
    ct = (valid.float() / valid.sum()).contiguous()  # cotangent of the masked mean

    def step():
        hd.grad = None
        nll, _, _ = L.kernel_forward_parts(hd, head, t, ignore_index=IGNORE)
        nll.backward(ct)

    sec = time_region(step, steps, warmup)

    # Roofline kernel: the forward launch (lce_fwd_kernel + its finalize), one event pair per launch on
    # the stream it is launched on; the mean over `steps` launches is the figure the roofline uses
    # (the median is reported beside it).
    fwd_ms = event_ms(_fwd_launcher(h.contiguous(), head, t.contiguous(), head_kind), steps, warmup=1)

    # Per-phase durations, events on the launch stream: [fwd][bwd] per step.
    stream = torch.cuda.current_stream()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        hd.grad = None
        evs[i][0].record(stream)
        nll, _, _ = L.kernel_forward_parts(hd, head, t, ignore_index=IGNORE)
        evs[i][1].record(stream)
        nll.backward(ct)
        evs[i][2].record(stream)
    torch.cuda.synchronize()
    phase_fwd = statistics.median(e[0].elapsed_time(e[1]) for e in evs)
    phase_bwd = statistics.median(e[1].elapsed_time(e[2]) for e in evs)

    # Loss-layer memory, the worker's way: the forward's marginal peak, then the backward's (G chunk
    # + dH; the transposed head is already cached by the warm-up and reported on its own).
    hd.grad = None
    torch.cuda.empty_cache()
    fwd_peak, (nll, _, _) = marginal_peak_bytes(lambda: L.kernel_forward_parts(hd, head, t, ignore_index=IGNORE))
    bwd_peak, _ = marginal_peak_bytes(lambda: nll.backward(ct))
    del nll
    copy = os.environ.get("MTP_LCE_TRANSPOSED_HEAD", "auto")
    staged = ((copy == "0" or (head_kind == "q4" and copy != "1"))
              and os.environ.get("MTP_LCE_STAGE_HEAD", "1") != "0")
    fwd_staged = (head_kind == "q4" and os.environ.get("MTP_LCE_STAGE_HEAD", "1") != "0"
                  and plan.lce_fwd_stages_whole_head(N, D, V, plan.lce_bwd_budget_bytes()))
    p = plan.lce_plan(n=N, v=V, d=D, staged=staged, quantized=head_kind == "q4", fwd_staged=fwd_staged)
    head_t = L.transposed_head_cache_bytes()
    return {"sec_per_step": sec, "fwd_ms": phase_fwd, "bwd_ms": phase_bwd,
            "fwd_kernel_ms_median": statistics.median(fwd_ms), "fwd_kernel_ms_mean": sum(fwd_ms) / len(fwd_ms),
            "fwd_kernel_launches": len(fwd_ms),
            "fwd_marginal_peak_gb": fwd_peak / 1e9, "bwd_marginal_peak_gb": bwd_peak / 1e9,
            "fwd_workspace_gb": p.fwd_workspace_bytes / 1e9,
            "bwd_workspace_gb": p.bwd_workspace_bytes / 1e9, "bwd_row_block": p.bwd_row_block,
            "bwd_row_blocks": p.bwd_row_blocks, "bwd_chunk": p.bwd_chunk, "bwd_chunks": p.bwd_chunks,
            "transposed_head_cache_gb": head_t / 1e9,
            "bwd_footprint_gb": (bwd_peak + head_t) / 1e9}


def bench_trainable_lce(steps, warmup):
    """LCE fwd+bwd with a trainable dense head at the flagship shape: dL/dH and dL/dW (the dW kernel,
    one owner per (vocab, hidden) output tile). Four vocab-tile products per step (forward logits;
    backward logits, dH and dW), 2 N V D flops each. The head's backward stages its transposed vocab
    chunks in the workspace (the default for a trainable head, whose cached copy an optimizer step
    would invalidate; this loop takes no optimizer step)."""
    import torch

    from mlx_train_perf.core import loss as L
    from mlx_train_perf.core.loss import DenseHead

    h, w, t = lce_inputs_gpu(N, D, V)
    wd = w.detach().requires_grad_(True)
    head = DenseHead(weight=wd, trainable=True)
    hd = h.detach().requires_grad_(True)
    valid = (t != IGNORE)
    ct = (valid.float() / valid.sum()).contiguous()

    def step():
        hd.grad = None
        wd.grad = None
        nll, _, _ = L.kernel_forward_parts(hd, head, t, ignore_index=IGNORE)
        nll.backward(ct)

    sec = time_region(step, steps, warmup)
    hd.grad = None
    wd.grad = None
    torch.cuda.empty_cache()
    nll, _, _ = L.kernel_forward_parts(hd, head, t, ignore_index=IGNORE)
    bwd_peak, _ = marginal_peak_bytes(lambda: nll.backward(ct))
    flops = 4 * 2.0 * N * V * D
    return {"ms_per_step": sec * 1e3, "tokens_per_s": N / sec, "step_tflops": flops / sec / 1e12,
            "step_mfma_frac": flops / sec / 1e12 / PEAK_BF16_TFLOPS, "bwd_marginal_peak_gb": bwd_peak / 1e9,
            "products_per_step": 4}


def lce_footprint_curve(steps=6):
    """The backward's memory / time trade at the flagship: the step and its backward footprint
    (marginal peak + the cached transposed head) for workspace budgets of 3, 1.5 (default) and 0.75
    GiB; without the transposed head (MTP_LCE_TRANSPOSED_HEAD=0: each vocab chunk of the head staged,
    transposed, in the workspace) at 1.5 and 0.75 GiB; and with neither copy nor staging
    (MTP_LCE_STAGE_HEAD=0: the dH product reads W through LDS transpose reads)."""
    import torch

    from mlx_train_perf.core import loss as L

    out = {}
    saved = {k: os.environ.get(k) for k in ("MTP_LCE_BWD_BUDGET", "MTP_LCE_TRANSPOSED_HEAD", "MTP_LCE_STAGE_HEAD")}
    cases = (("budget_3gib", {"MTP_LCE_BWD_BUDGET": str(3 << 30)}), ("budget_1_5gib_default", {}),
             ("budget_0_75gib", {"MTP_LCE_BWD_BUDGET": str(3 << 28)}),
             ("no_head_copy", {"MTP_LCE_TRANSPOSED_HEAD": "0"}),
             ("no_head_copy_0_75gib", {"MTP_LCE_TRANSPOSED_HEAD": "0", "MTP_LCE_BWD_BUDGET": str(3 << 28)}),
             ("no_head_copy_transposed_reads", {"MTP_LCE_TRANSPOSED_HEAD": "0", "MTP_LCE_STAGE_HEAD": "0"}))
    try:
        for name, env in cases:
            for k, val in saved.items():   # each case starts from the caller's settings
                if val is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = val
            os.environ.update(env)
            L.clear_transposed_head_cache()
            torch.cuda.empty_cache()
            r = bench_lce(steps, 1, "dense")
            out[name] = {"ms_per_step": r["sec_per_step"] * 1e3, "bwd_row_blocks": r["bwd_row_blocks"],
                         "bwd_chunks": r["bwd_chunks"], "bwd_marginal_peak_gb": r["bwd_marginal_peak_gb"],
                         "transposed_head_cache_gb": r["transposed_head_cache_gb"],
                         "bwd_footprint_gb": r["bwd_footprint_gb"]}
    finally:
        for k, val in saved.items():
            if val is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = val
        L.clear_transposed_head_cache()
    return out


def bench_lce_fp32_c1(steps, warmup):
    """BASELINE config 1 in fp32 on the GPU (N=1024, D=512, V=32000, 10% ignore_index): the fp32
    entry points (fp32 MFMA), fwd+bwd per step, beside the fp32 CPU baseline of the same config."""
    import torch

    from mlx_train_perf.core import loss as L
    from mlx_train_perf.core.loss import DenseHead

    g = torch.Generator(device="cuda").manual_seed(0)
    n, d, v = 1024, 512, 32000
    h = torch.randn(n, d, generator=g, device="cuda")
    w = torch.randn(v, d, generator=g, device="cuda") * 0.02
    t = torch.randint(0, v, (n,), generator=g, device="cuda")
    t[torch.randperm(n, generator=g, device="cuda")[:102]] = IGNORE
    head = DenseHead(weight=w, trainable=False)
    hd = h.requires_grad_(True)
    valid = t != IGNORE
    ct = (valid.float() / valid.sum()).contiguous()

    def step():
        hd.grad = None
        nll, _, _ = L.kernel_forward_parts(hd, head, t, ignore_index=IGNORE)
        nll.backward(ct)

    sec = time_region(step, steps, warmup)
    flops = 6.0 * n * v * d
    return {"ms_per_step": sec * 1e3, "tokens_per_s": n / sec, "tflops": flops / sec / 1e12,
            "fp32_mfma_frac": flops / sec / 1e12 / PEAK_FP32_TFLOPS, "dtype": "fp32 (fp32 MFMA)"}


def lce_ladder(reps=10):
    """Forward loss layer at n in {512, 2048, 8192} (D=4096, V=151936): the fused kernel against the
    same-device naive path (full bf16 logits, fp32 logsumexp; core/naive.py), the reference's
    kernel-vs-naive gate being <= 1.7x (scripts/bench_loss_layer.py:44-51); plus the fused fwd+bwd."""
    import torch

    from mlx_train_perf.core import loss as L
    from mlx_train_perf.core.naive import naive_linear_ce

    out = {}
    _, w, _ = lce_inputs_gpu(8, D, V, seed=1)
    head = L.DenseHead(weight=w, trainable=False)
    for n in (512, 2048, 8192):
        h, _, t = lce_inputs_gpu(n, D, V, seed=n)
        ts = torch.where(t == IGNORE, torch.zeros_like(t), t)
        k_ms = statistics.median(event_ms(_fwd_launcher(h, head, t, "dense"), reps))
        naive_ms = statistics.median(event_ms(lambda: naive_linear_ce(h, w, ts), max(3, reps // 2)))
        torch.cuda.empty_cache()
        k_peak, _ = marginal_peak_bytes(lambda: L.kernel_forward_parts(h, head, t, ignore_index=IGNORE))
        n_peak, _ = marginal_peak_bytes(lambda: naive_linear_ce(h, w, ts))
        hd = h.detach().requires_grad_(True)
        ct = torch.full((n,), 1.0 / n, device="cuda")

        def fb():
            hd.grad = None
            nll, _, _ = L.kernel_forward_parts(hd, head, t, ignore_index=IGNORE)
            nll.backward(ct)

        fb_ms = statistics.median(event_ms(fb, reps))
        out[f"n{n}"] = {"fwd_kernel_ms": k_ms, "fwd_naive_ms": naive_ms, "kernel_over_naive": k_ms / naive_ms,
                        "fwd_kernel_peak_gb": k_peak / 1e9, "fwd_naive_peak_gb": n_peak / 1e9,
                        "fwd_tflops": 2.0 * n * V * D / (k_ms * 1e-3) / 1e12,
                        "fwdbwd_kernel_ms": fb_ms, "fwdbwd_tflops": 6.0 * n * V * D / (fb_ms * 1e-3) / 1e12}
        del h, t, ts, hd
        torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------------------------------------
# Attention (configs 4, 5)
# ------------------------------------------------------------------------------------------------
def _attn_inputs(s, seed=0, b=ATT_B, dh=ATT_DH):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    mk = lambda h: torch.randn(b, h, s, dh, generator=g, device="cuda").to(torch.bfloat16)  # noqa: E731
    return mk(ATT_HQ), mk(ATT_HKV), mk(ATT_HKV), mk(ATT_HQ)


def bench_attention(steps, warmup, mode="causal", s=None, dh=ATT_DH, fp32=False):
    """Flash attention fwd and fwd+bwd at B=1, Hq=32, Hkv=8, head_dim `dh` (128: configs 4, 5). mode:
    "causal" (config 4, S=8192), "packed" (config 5, S=16384, seeded document lengths), "full"
    (non-causal, S=8192). `fp32`: the same inputs in fp32 on the fp32 kernels, rated against the fp32
    MFMA peak."""
    import torch

    from mlx_train_perf.attention.api import kernel_backward, kernel_forward
    from mlx_train_perf.plan import launch as plan

    s = s or (16384 if mode == "packed" else 8192)
    q, k, v, do = _attn_inputs(s, dh=dh)
    if fp32:
        q, k, v, do = (x.float() for x in (q, k, v, do))
    scale = 1.0 / math.sqrt(dh)
    sid = sst = None
    causal = mode != "full"
    if mode == "packed":
        lens = packed_lengths(s)
        ids, starts, pos = [], [], 0
        for i, n_ in enumerate(lens):
            ids += [i] * n_
            starts += [pos] * n_
            pos += n_
        sid = torch.tensor([ids], dtype=torch.int32, device="cuda")
        sst = torch.tensor([starts], dtype=torch.int32, device="cuda")
        pairs = plan.packed_pairs(lens)
    elif mode == "full":
        pairs = s * s
    else:
        pairs = plan.causal_pairs(s)
    state = {}

    def fwd():
        state["o"], state["l"] = kernel_forward(q, k, v, scale=scale, seg_id=sid, seg_start=sst, causal=causal)
        return state["o"]

    def fwdbwd():
        fwd()
        return kernel_backward(q, k, v, state["o"], state["l"], do, scale=scale, seg_id=sid, seg_start=sst,
                               causal=causal)

    fwd_s = time_region(fwd, steps, warmup)
    fb_s = time_region(fwdbwd, steps, warmup)
    state.clear()
    torch.cuda.empty_cache()
    fwd_peak, _ = marginal_peak_bytes(fwd)
    state.clear()
    torch.cuda.empty_cache()
    fb_peak, _ = marginal_peak_bytes(fwdbwd)
    state.clear()
    flops_fwd = 2.0 * 2 * dh * ATT_HQ * ATT_B * pairs
    flops_fb = 2.0 * 7 * dh * ATT_HQ * ATT_B * pairs
    out = {"seq": s, "fwd_ms": fwd_s * 1e3, "fwdbwd_ms": fb_s * 1e3, "bwd_ms": (fb_s - fwd_s) * 1e3,
           "pairs_per_head": pairs, "algorithmic_tflop": flops_fb / 1e12,
           "fwd_tflops": flops_fwd / fwd_s / 1e12, "tflops": flops_fb / fb_s / 1e12,
           "mfma_frac": flops_fb / fb_s / 1e12 / (PEAK_FP32_TFLOPS if fp32 else PEAK_BF16_TFLOPS),
           "fwd_marginal_peak_gb": fwd_peak / 1e9, "fwdbwd_marginal_peak_gb": fb_peak / 1e9}
    if mode == "packed":
        out["segments"] = len(lens)
        out["tile_efficiency"] = attention_tile_efficiency(lens, s)
    elif mode == "causal":
        out["tile_efficiency"] = attention_tile_efficiency(None, s)
    return out


def attention_tile_efficiency(lens: list[int] | None, s: int) -> dict:
    """Visible (query, key) pairs / pairs in the tiles the head_dim-128 kernels visit, per head, for
    a packed layout (`lens`) or the causal mask (None). Forward and dQ: a 32-query wave block visits
    the 64-key tiles from its workgroup's first segment start (rounded down to 64) up to its last
    query. dK/dV: a 128-key block visits the 64-query tiles from its first key (rounded down) up to
    the end of its last key's segment."""
    import bisect

    if lens is None:
        lens = [s]
    starts, pos = [], 0
    for n in lens:
        starts += [pos] * n
        pos += n
    visible = sum(n * (n + 1) // 2 for n in lens)
    fwd = 0
    for q0 in range(0, s, 32):
        q1 = min(q0 + 32, s)
        kv0 = starts[q0] // 64 * 64
        fwd += 32 * 64 * (-(-(q1 - kv0) // 64))
    dkv = 0
    for k0 in range(0, s, 128):
        klast = min(k0 + 127, s - 1)
        q_end = bisect.bisect_right(starts, klast)   # first position whose segment starts past klast
        q_begin = k0 // 64 * 64
        dkv += 128 * 64 * max(0, -(-(q_end - q_begin) // 64))
    return {"visible_pairs": visible, "fwd_dq_visited_pairs": fwd, "dkv_visited_pairs": dkv,
            "fwd_dq_efficiency": visible / fwd, "dkv_efficiency": visible / dkv}


def attention_ladder(steps, warmup):
    """Causal fwd and fwd+bwd at S in {2048, 4096, 8192} (the reference publishes all three,
    community-benchmarks flash_n2048 / n4096 / n8192)."""
    out = {}
    for s in (2048, 4096, 8192):
        r = bench_attention(steps, warmup, "causal", s=s)
        out[f"s{s}"] = {k: r[k] for k in ("fwd_ms", "fwdbwd_ms", "fwd_tflops", "tflops", "mfma_frac")}
    return out


def attention_headdim_ladder(steps, warmup):
    """Causal fwd and fwd+bwd at S=8192, 32/8 heads, head_dim 64 and 96 (the other head dims the
    reference's kernels take, src/mlx_train_perf/attention/api.py:107-110; 128 is config 4 itself)."""
    out = {}
    for dh in (64, 96):
        r = bench_attention(steps, warmup, "causal", dh=dh)
        out[f"d{dh}"] = {k: r[k] for k in ("fwd_ms", "fwdbwd_ms", "fwd_tflops", "tflops", "mfma_frac")}
    return out


# ------------------------------------------------------------------------------------------------
# CPU baselines: the oracle (PyTorch-CPU fp32 restatement of the reference's naive / stock paths) on
# the GPU box's host cores, median of 3 after one warm-up (bench/worker.py:121-133).
# ------------------------------------------------------------------------------------------------
def _cpu_threads():
    import torch

    if "OMP_NUM_THREADS" not in os.environ:  # the GPU box sets it to its CPU share
        torch.set_num_threads(os.cpu_count() or 1)
    return torch.get_num_threads()


def _median_runs(run, reps=3):
    run(warm=True)
    ts = [run(warm=False) for _ in range(reps)]
    return statistics.median(ts), ts


def cpu_baseline_lce(budget_s: float = 4.0):
    """Flagship LCE fwd+bwd (full D, V) on a bounded sample of the 8192 tokens."""
    import torch

    from oracle import lce as olce

    cores = _cpu_threads()
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(V, D, generator=g) * 0.02).to(torch.bfloat16).to(torch.float32)  # bf16 values, fp32 storage

    def sample(rows):
        h = torch.randn(rows, D, generator=g)
        h = (h / torch.sqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
        return h, torch.randint(0, V, (rows,), generator=g)

    def timed(h, t):
        t0 = time.perf_counter()
        _, lse, _ = olce.forward(h, w, t, ignore_index=IGNORE, dtype=torch.float32)
        olce.backward(h, w, t, lse, torch.full((t.shape[0],), 1.0 / t.shape[0]), ignore_index=IGNORE,
                      dtype=torch.float32)
        return time.perf_counter() - t0

    timed(*sample(8))
    probe = 256
    dt = timed(*sample(probe))
    rows = int(max(64, min(N, probe * budget_s / max(dt, 1e-3))))
    h, t = sample(rows)
    med, ts = _median_runs(lambda warm: timed(h, t) if not warm else timed(*sample(8)))
    return {"value": rows / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"LCE fwd+bwd on {rows} of the {N} tokens (D={D}, V={V}), oracle/lce.py fp32, median of "
                      f"{len(ts)} runs ({', '.join(f'{x:.2f}' for x in ts)} s); CPU {_cpu_model()}",
            "reps": len(ts)}


def cpu_baseline_c1():
    """Config 1 in full: N=1024, D=512, V=32000 fp32, 10% ignore_index, fwd+bwd."""
    import torch

    from oracle import lce as olce

    cores = _cpu_threads()
    n, d, v = 1024, 512, 32000
    g = torch.Generator().manual_seed(1)
    h = torch.randn(n, d, generator=g)
    w = torch.randn(v, d, generator=g) * 0.02
    t = torch.randint(0, v, (n,), generator=g)
    t[torch.randperm(n, generator=g)[: round(0.1 * n)]] = IGNORE
    valid = t != IGNORE

    def run(warm):
        t0 = time.perf_counter()
        _, lse, _ = olce.forward(h, w, t, ignore_index=IGNORE, dtype=torch.float32)
        olce.backward(h, w, t, lse, valid.float() / valid.sum(), ignore_index=IGNORE, round_g_bf16=False,
                      dtype=torch.float32)
        return time.perf_counter() - t0

    med, ts = _median_runs(run)
    return {"value": n / med, "unit": "tokens/s", "ms": med * 1e3, "tflops": 6.0 * n * v * d / med / 1e12,
            "cores": cores, "kind": "port", "reps": len(ts),
            "sample": f"config 1 in full (N={n}, D={d}, V={v}, fp32, 10% ignore), oracle/lce.py, median of "
                      f"{len(ts)}; CPU {_cpu_model()}"}


def cpu_baseline_attention(max_s: float = 6.0):
    """Config 4 on one kv-head group (4 query heads, S=8192, head_dim 128), fp32, materialized scores
    and the FlashAttention backward equations (oracle/attention.py); the full config is 8 groups."""
    import torch

    from oracle import attention as oatt
    from mlx_train_perf.plan import launch as plan

    cores = _cpu_threads()
    s, grp = 8192, ATT_HQ // ATT_HKV
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, grp, s, ATT_DH, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 1, s, ATT_DH, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 1, s, ATT_DH, generator=g).to(torch.bfloat16)
    do = torch.randn(1, grp, s, ATT_DH, generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(ATT_DH)

    def run(warm):
        qq, kk, vv, dd = (x[..., : 256, :] if warm else x for x in (q, k, v, do))
        t0 = time.perf_counter()
        o, lse = oatt.attention_forward(qq, kk, vv, scale=scale, dtype=torch.float32)
        oatt.attention_backward(qq, kk, vv, o, lse, dd, scale=scale, dtype=torch.float32)
        return time.perf_counter() - t0

    run(True)
    first = run(False)
    ts = [first] + ([run(False), run(False)] if first < max_s else [])
    med = statistics.median(ts)
    flop = 2.0 * 7 * ATT_DH * grp * plan.causal_pairs(s)
    return {"value": med * 1e3, "unit": "ms per kv-head group", "full_config_ms": 8 * med * 1e3,
            "tflops": flop / med / 1e12, "cores": cores, "kind": "port", "reps": len(ts),
            "sample": f"config 4 on 1 of its 8 kv-head groups (Hq=4, Hkv=1, S={s}, d={ATT_DH}), fp32, oracle/"
                      f"attention.py fwd+bwd, {'median of 3' if len(ts) == 3 else 'one run (reps=1)'}; "
                      f"CPU {_cpu_model()}"}


# ------------------------------------------------------------------------------------------------
# Profiles. `--pmc-workload` is the program the rocprofv3 --pmc passes profile; `--pmc-summary`
# merges the passes' counter csv files into the markdown committed under profiles/, whose json
# block committed_traffic() reads back. Traffic: FETCH_SIZE / WRITE_SIZE (KiB per dispatch) scaled
# by what they read for a 1 GiB device copy in the same run. MFMA: SQ_VALU_MFMA_BUSY_CYCLES over
# 4 x SQ_BUSY_CU_CYCLES (reads ~1.0 on the register-only MFMA loop of mtp_bench_mfma_ceiling, which
# the workload runs as the calibration), SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 = executed bf16 flop.
# ------------------------------------------------------------------------------------------------
PMC_COPY_BYTES = 1 << 30
PMC_PROFILE = ROOT / "profiles" / "pmc_bench_workload_traffic_mfma.md"


def committed_traffic(kernel: str):
    try:
        text = PMC_PROFILE.read_text()
        blob = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(blob)["kernels"][kernel]["traffic_bytes"]
    except (OSError, IndexError, KeyError, ValueError):
        return None


def pmc_workload():
    """One pass of each profiled workload (no timing): the 1 GiB copy and the MFMA loop
    (calibrations), the flagship LCE forward + backward (dense, and 4-bit dequantized in registers),
    causal attention (S=8192) and packed attention (S=16384, config 5). Each kernel instantiation
    serves one workload here, so per-kernel counter means are per-workload figures (non-causal
    attention would share the causal instantiations, and is left out; so would the staged 4-bit
    path, whose products are the dense instantiations over dequantized rows, so the 4-bit pass runs
    with MTP_LCE_STAGE_HEAD=0)."""
    import torch

    from mlx_train_perf import _native
    from mlx_train_perf.attention.api import kernel_backward, kernel_forward
    from mlx_train_perf.core.loss import kernel_forward_parts

    x = torch.empty(PMC_COPY_BYTES // 2, dtype=torch.int16, device="cuda").fill_(1)
    y = torch.empty_like(x)
    for _ in range(2):
        y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    out = torch.zeros(1024, device="cuda")
    _native.load().mtp_bench_mfma_ceiling(1024, 2000, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    print("pmc workload: calibrations done", flush=True)
    for kind in ("dense", "q4"):
        h, w, t = lce_inputs_gpu(N, D, V)
        head = _lce_head(w, kind)
        hd = h.requires_grad_(True)
        saved = os.environ.get("MTP_LCE_STAGE_HEAD")
        if kind == "q4":
            os.environ["MTP_LCE_STAGE_HEAD"] = "0"
        try:
            for _ in range(2):
                nll, _, _ = kernel_forward_parts(hd, head, t, ignore_index=IGNORE)
                nll.backward(torch.full_like(nll, 1.0 / N))
            torch.cuda.synchronize()
        finally:
            if saved is None:
                os.environ.pop("MTP_LCE_STAGE_HEAD", None)
            else:
                os.environ["MTP_LCE_STAGE_HEAD"] = saved
        del h, w, t, hd, head
        torch.cuda.empty_cache()
        print(f"pmc workload: lce {kind} done", flush=True)
    for mode in ("causal", "packed"):
        s = 16384 if mode == "packed" else 8192
        q, k, v, do = _attn_inputs(s)
        sid = sst = None
        if mode == "packed":
            lens = packed_lengths(s)
            sid = torch.tensor([sum(([i] * n for i, n in enumerate(lens)), [])], dtype=torch.int32, device="cuda")
            starts, pos = [], 0
            for n in lens:
                starts += [pos] * n
                pos += n
            sst = torch.tensor([starts], dtype=torch.int32, device="cuda")
        for _ in range(2):
            o, l = kernel_forward(q, k, v, scale=1 / math.sqrt(ATT_DH), seg_id=sid, seg_start=sst,
                                  causal=mode != "full")
            kernel_backward(q, k, v, o, l, do, scale=1 / math.sqrt(ATT_DH), seg_id=sid, seg_start=sst,
                            causal=mode != "full")
        torch.cuda.synchronize()
        print(f"pmc workload: attention {mode} done", flush=True)
    print("pmc workload done", flush=True)


def _pmc_dispatches(root: str) -> dict:
    """kernel -> counter -> {dispatch id: value summed over the counter's dimension rows}."""
    import collections
    import csv
    import glob
    import re

    acc = collections.defaultdict(lambda: collections.defaultdict(lambda: collections.defaultdict(float)))
    for f in glob.glob(f"{root}/**/*counter_collection.csv", recursive=True):
        with open(f) as fh:
            for row in csv.DictReader(fh):
                name = re.sub(r"\(.*", "", row["Kernel_Name"]).replace("void ", "").strip()
                acc[name][row["Counter_Name"]][row["Dispatch_Id"]] += float(row["Counter_Value"])
    return acc


def pmc_summary(command: str, *dirs: str) -> str:
    merged: dict = {}
    for d in dirs:
        for k, cs in _pmc_dispatches(d).items():
            merged.setdefault(k, {}).update(cs)
    mean = {k: {c: sum(v.values()) / len(v) for c, v in cs.items()} for k, cs in merged.items()}
    calls = {k: max(len(v) for v in cs.values()) for k, cs in merged.items()}
    copy = [k for k in merged if "copyBuffer" in k]   # the runtime's blit kernel: the 1 GiB copy
    cal = {}
    if any("FETCH_SIZE" in merged[k] for k in copy):
        cf = max(max(merged[k]["FETCH_SIZE"].values()) for k in copy if "FETCH_SIZE" in merged[k])
        cw = max(max(merged[k]["WRITE_SIZE"].values()) for k in copy if "WRITE_SIZE" in merged[k])
        cal.update(copy_bytes=PMC_COPY_BYTES, fetch_kib=cf, write_kib=cw,
                   fetch_factor=PMC_COPY_BYTES / (cf * 1024.0), write_factor=PMC_COPY_BYTES / (cw * 1024.0))
    if any("TCC_EA0_RDREQ_DRAM_32B_sum" in merged[k] for k in copy):
        cd = max(max(merged[k]["TCC_EA0_RDREQ_DRAM_32B_sum"].values()) for k in copy
                 if "TCC_EA0_RDREQ_DRAM_32B_sum" in merged[k])
        cal.update(dram_read_32b=cd, dram_read_factor=PMC_COPY_BYTES / (cd * 32.0))
        big = max((k for k in copy if "TCC_EA0_RDREQ_DRAM_32B_sum" in merged[k]),
                  key=lambda k: max(merged[k]["TCC_EA0_RDREQ_DRAM_32B_sum"].values()))
        m = mean[big]
        if m.get("TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum") is not None and m.get("GRBM_GUI_ACTIVE"):
            cal["copy_read_credit_stall_frac"] = m["TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum"] / (16.0 * m["GRBM_GUI_ACTIVE"])
    ceil = next((k for k in merged if "mfma_ceiling" in k), None)
    if ceil and "SQ_VALU_MFMA_BUSY_CYCLES" in mean[ceil]:
        c = mean[ceil]
        cal["mfma_busy_ceiling_kernel"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * c["SQ_BUSY_CU_CYCLES"])
    algorithmic_bytes = {   # bytes that must cross HBM at least once per launch
        "lce_fwd_kernel<0>": 2.0 * (V * D + N * D),
        "lce_fwd_kernel<1>": 0.5 * V * D + 4.0 * V * D / 64 + 2.0 * N * D,
        "attn_kv_kernel<128, false, false>": 2.0 * (32 + 2 * 8) * 8192 * 128 + 4.0 * 32 * 8192 + 2.0 * 32 * 8192 * 128,
    }
    kernels = {}
    for k in sorted(merged):
        if not k.startswith("mtp::"):
            continue
        m, r = mean[k], {"dispatches": calls[k]}
        if "FETCH_SIZE" in m and "fetch_factor" in cal:
            r["fetch_bytes"] = m["FETCH_SIZE"] * 1024.0 * cal["fetch_factor"]
            r["write_bytes"] = m.get("WRITE_SIZE", 0.0) * 1024.0 * cal["write_factor"]
            r["traffic_bytes"] = r["fetch_bytes"] + r["write_bytes"]
        if "SQ_VALU_MFMA_BUSY_CYCLES" in m and m.get("SQ_BUSY_CU_CYCLES"):
            r["mfma_busy"] = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * m["SQ_BUSY_CU_CYCLES"])
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in m:
            r["executed_bf16_tflop"] = m["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512.0 / 1e12
        if "GRBM_GUI_ACTIVE" in m:
            r["gui_active_cycles"] = m["GRBM_GUI_ACTIVE"]
        if "TCC_EA0_RDREQ_DRAM_32B_sum" in m:
            r["dram_read_bytes"] = m["TCC_EA0_RDREQ_DRAM_32B_sum"] * 32.0
        if "TCC_EA0_WRREQ_DRAM_sum" in m:
            r["dram_write_requests"] = m["TCC_EA0_WRREQ_DRAM_sum"]
        if "TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum" in m and m.get("GRBM_GUI_ACTIVE"):
            # GRBM_GUI_ACTIVE sums the 8 XCDs' cycles; each XCD has 16 L2 channels
            r["dram_read_credit_stall_frac"] = m["TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum"] / (16.0 * m["GRBM_GUI_ACTIVE"])
        short = k[len("mtp::"):]
        if short in algorithmic_bytes:
            r["algorithmic_bytes"] = algorithmic_bytes[short]
        kernels[short] = r
    lines = ["# Counters per launch: bench.py --pmc-workload (LCE N=8192 D=4096 V=151936 dense <0> and 4-bit dequantized in registers <1>; "
             "attention S=8192 causal <false, *>, S=16384 packed <true, *>)", "",
             "Commands (repository root on the GPU box; one rocprofv3 pass per counter group):", "", "```", command,
             "```", ""]
    if "fetch_factor" in cal:
        lines += [f"Traffic calibration: a {PMC_COPY_BYTES} B device copy read FETCH_SIZE={cal['fetch_kib']:.0f} KiB "
                  f"and WRITE_SIZE={cal['write_kib']:.0f} KiB per dispatch, so bytes = KiB x 1024 x "
                  f"{cal['fetch_factor']:.4f} (fetch) and x {cal['write_factor']:.4f} (write).", ""]
    if "mfma_busy_ceiling_kernel" in cal:
        lines += ["MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (4 x SQ_BUSY_CU_CYCLES); the register-only MFMA loop "
                  f"(`mfma_ceiling_kernel`) reads {cal['mfma_busy_ceiling_kernel']:.3f}. Executed bf16 TFLOP = "
                  "SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512.", ""]
    if "dram_read_factor" in cal:
        lines += [f"DRAM side: TCC_EA0_RDREQ_DRAM_32B_sum counts the L2's read requests to the memory side in "
                  f"32-byte units; the same copy read {cal['dram_read_32b']:.0f} of them "
                  f"({cal['dram_read_32b'] * 32 / PMC_COPY_BYTES:.4f} x its bytes). The memory-side cache (MALL) "
                  "sits behind that interface, so these bytes still include MALL hits: no counter exposed on "
                  "this image separates MALL from HBM. Read credit stall = "
                  "TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum / (16 channels x GRBM_GUI_ACTIVE): the fraction of L2 "
                  "channel cycles that waited for memory-side read credits"
                  + (f". The HBM-bound copy reads {cal['copy_read_credit_stall_frac']:.3f}, so a low value does "
                     "not show memory-side headroom; only high values mean much."
                     if "copy_read_credit_stall_frac" in cal else "."), ""]
    lines += ["| kernel | dispatches | fetch GB | write GB | traffic GB | algorithmic GB | DRAM-side read GB | "
              "read credit stall | MFMA busy | executed bf16 TFLOP |",
              "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]

    def f(x, scale=1e9, fmt="{:.3f}"):
        return "" if x is None else fmt.format(x / scale)

    for k, r in kernels.items():
        lines.append(f"| `{k}` | {r['dispatches']} | {f(r.get('fetch_bytes'))} | {f(r.get('write_bytes'))} | "
                     f"{f(r.get('traffic_bytes'))} | {f(r.get('algorithmic_bytes'))} | "
                     f"{f(r.get('dram_read_bytes'))} | {f(r.get('dram_read_credit_stall_frac'), 1, '{:.3f}')} | "
                     f"{f(r.get('mfma_busy'), 1, '{:.3f}')} | {f(r.get('executed_bf16_tflop'), 1, '{:.3f}')} |")
    blob = {"calibration": cal, "kernels": kernels}
    lines += ["", "```json", json.dumps(blob, indent=1), "```", ""]
    return "\n".join(lines)


def trace_summary(trace_csv: str, title: str, command: str, stats_csv: str | None = None) -> str:
    """Markdown table of this library's kernels from a rocprofv3 --kernel-trace csv (one row per
    dispatch), one line per (kernel, grid size) -- i.e. per launch shape, since the ladders reuse the
    kernels at other sizes: calls, median, mean, the mean without the shape's first dispatch (its
    warm-up), min and max. With the same run's --stats csv, its per-kernel calls and average too."""
    import collections
    import csv
    import re

    durs = collections.defaultdict(list)
    for r in sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"])):
        if "mtp::" in r["Kernel_Name"]:
            name = re.sub(r"\(.*", "", r["Kernel_Name"]).replace("void ", "").replace("mtp::", "").strip()
            grid = int(r.get("Grid_Size") or r.get("Grid_Size_X") or 0)
            durs[(name, grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = [f"# {title}", "", "Command (repository root on the GPU box):", "", "```", command, "```", "",
           "Per-launch-shape durations from `rocprofv3 --kernel-trace` (one row per dispatch), microseconds; "
           "grid = work-items. The bench line's roofline uses the mean of its per-launch event times (which "
           "also hold the forward's 22 us finalize launch); compare it with the mean here.", "",
           "| kernel | grid | calls | median us | mean us | mean w/o first us | min us | max us |",
           "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for (name, grid), d in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
        rest = d[1:] or d
        out.append(f"| `{name}` | {grid} | {len(d)} | {statistics.median(d):.1f} | {sum(d) / len(d):.1f} | "
                   f"{sum(rest) / len(rest):.1f} | {min(d):.1f} | {max(d):.1f} |")
    if stats_csv:
        out += ["", "`rocprofv3 --stats` of the same run (all launch shapes of a kernel together), microseconds:", "",
                "| kernel | calls | average us | min us | max us |", "|---|---:|---:|---:|---:|"]
        for r in csv.DictReader(open(stats_csv)):
            if "mtp::" in r["Name"]:
                name = re.sub(r"\(.*", "", r["Name"]).replace("void ", "").replace("mtp::", "").strip()
                out.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                           f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} |")
    return "\n".join(out) + "\n"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--pmc-workload", action="store_true", help="run the profiled workloads once (no timing)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="ARG",
                    help="COMMAND DIR [DIR ...]: summarize rocprofv3 --pmc csv outputs into markdown")
    ap.add_argument("--trace-summary", nargs="+", metavar="ARG",
                    help="TRACE_CSV TITLE COMMAND [STATS_CSV]: summarize a rocprofv3 --kernel-trace csv (and the "
                         "same run's --stats csv) into markdown")
    ap.add_argument("--parts", default="lce,qlora,trainable,attention,ladder,footprint,fp32",
                    help="comma list of lce, qlora, trainable, attention, ladder, footprint, fp32 (lce is the "
                         "headline line)")
    args = ap.parse_args()
    if args.pmc_summary:
        print(pmc_summary(*args.pmc_summary))
        return
    if args.trace_summary:
        print(trace_summary(*args.trace_summary), end="")
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (this build runs on one GPU; "
              "sharding across GPUs is a design here, not a measured configuration)", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.pmc_workload:
        pmc_workload()
        return

    lce = bench_lce(args.steps, args.warmup, "dense")
    sec = lce["sec_per_step"]
    flops_step = 6.0 * N * V * D
    fwd_flops = 2.0 * N * V * D
    ach = fwd_flops / (lce["fwd_kernel_ms_mean"] * 1e-3) / 1e12
    result = {
        "metric": "fused-LCE fwd+bwd tokens/s @N8192 V151936 D4096 (bf16, frozen head)",
        "value": N / sec,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded: H~N(0,1) RMS-normalized, W~N(0,0.02), 5% ignore_index)",
        "config": {"workload": "lce_fwd_bwd_n8192_d4096_v151936_bf16_frozen_head", "tokens": N, "d": D, "v": V,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "kernel": "lce_fwd_kernel<0> (+ lce_fwd_finalize_kernel in the event window)",
                     "achieved": ach, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": ach / PEAK_BF16_TFLOPS,
                     "traffic": committed_traffic("lce_fwd_kernel<0>"),
                     "traffic_source": "profiles/pmc_bench_workload_traffic_mfma.md: rocprofv3 --pmc FETCH_SIZE + "
                                       "WRITE_SIZE of the same kernel and shape (a committed profile, not this run)",
                     "timing": f"mean of {lce['fwd_kernel_launches']} launches (after one warm-up), HIP events on "
                               "the launch stream; the window also holds the 22 us finalize launch"},
        "step_mfma_frac": flops_step / sec / 1e12 / PEAK_BF16_TFLOPS,
        "lce": {**lce, "step_tflops": flops_step / sec / 1e12},
    }
    try:
        result["mfma_ceiling_tflops"] = mfma_ceiling_tflops()
    except Exception as exc:  # measurement utility only
        result["mfma_ceiling_tflops"] = f"failed: {exc}"
    parts = set(args.parts.split(","))
    if not args.no_extras and "qlora" in parts:
        torch.cuda.empty_cache()
        q4 = bench_lce(max(3, args.steps // 4), 1, "q4")
        result["qlora_lce"] = {**q4, "tokens_per_s": N / q4["sec_per_step"],
                               "step_mfma_frac": flops_step / q4["sec_per_step"] / 1e12 / PEAK_BF16_TFLOPS}
        # The default 4-bit backward stages each vocab chunk of the head, dequantized and transposed,
        # in its workspace. The same step with the whole head kept as a cached bf16 transposed copy
        # (MTP_LCE_TRANSPOSED_HEAD=1), and with neither (MTP_LCE_STAGE_HEAD=0: the dH product
        # dequantizes the packed words in registers): the memory / time trades of the 4-bit backward.
        from mlx_train_perf.core import loss as L
        keys = ("MTP_LCE_TRANSPOSED_HEAD", "MTP_LCE_STAGE_HEAD")
        prev = {k: os.environ.get(k) for k in keys}
        runs = {}
        try:
            for name, copy, stage in (("head_copy", "1", "1"), ("in_register", "0", "0")):
                os.environ["MTP_LCE_TRANSPOSED_HEAD"] = copy
                os.environ["MTP_LCE_STAGE_HEAD"] = stage
                L.clear_transposed_head_cache()
                torch.cuda.empty_cache()
                q4n = bench_lce(3, 1, "q4")
                runs[name] = {"ms_per_step": q4n["sec_per_step"] * 1e3, "tokens_per_s": N / q4n["sec_per_step"],
                              "bwd_ms": q4n["bwd_ms"], "bwd_chunks": q4n["bwd_chunks"],
                              "bwd_marginal_peak_gb": q4n["bwd_marginal_peak_gb"],
                              "bwd_footprint_gb": q4n["bwd_footprint_gb"]}
        finally:
            # the user's settings (or their absence) hold for the parts that follow
            for k, val in prev.items():
                if val is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = val
        result["qlora_lce"].update(runs)
    if not args.no_extras and "trainable" in parts:
        torch.cuda.empty_cache()
        result["trainable_head_lce"] = bench_trainable_lce(max(3, args.steps // 4), 1)
    if not args.no_extras and "attention" in parts:
        torch.cuda.empty_cache()
        result["attention_causal_s8192"] = bench_attention(args.steps, args.warmup, "causal")
        result["attention_packed_s16384"] = bench_attention(args.steps, args.warmup, "packed")
        result["attention_noncausal_s8192"] = bench_attention(args.steps, args.warmup, "full")
    if not args.no_extras and "footprint" in parts:
        torch.cuda.empty_cache()
        result["lce_footprint"] = lce_footprint_curve()
    if not args.no_extras and "fp32" in parts:
        torch.cuda.empty_cache()
        result["lce_fp32_c1"] = bench_lce_fp32_c1(max(5, args.steps), 2)
        torch.cuda.empty_cache()
        result["attention_fp32_causal_s8192"] = bench_attention(3, 1, "causal", fp32=True)
    if not args.no_extras and "ladder" in parts:
        torch.cuda.empty_cache()
        result["lce_ladder_fwd"] = lce_ladder()
        result["attention_ladder_causal"] = attention_ladder(max(3, args.steps // 2), 2)
        result["attention_headdim_s8192"] = attention_headdim_ladder(max(3, args.steps // 2), 2)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_lce()
        result["cpu_baseline_c1"] = cpu_baseline_c1()
        result["cpu_baseline_attention"] = cpu_baseline_attention()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
