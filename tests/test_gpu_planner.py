"""GPU: the memory planner (plan/estimate.py `loss_bytes`) against the loss layer's measured marginal
peaks at BASELINE config 2 (N=8192, D=4096, V=151936, bf16), measured the reference worker's way
(bench/worker.py:117-132): reset the peak counter, run, max_memory_allocated minus what was allocated
before. Frozen head: the forward peak exactly; the backward peak = the planned workspace and dH, and
a first backward additionally the cached transposed head. Trainable head: the backward adds dL/dW and
takes every row in one block."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

N, D, V = 8192, 4096, 151936
IGN = -100


def _peak(fn):
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() - before, out


def _inputs():
    g = torch.Generator(device="cuda").manual_seed(0)
    h = torch.randn(N, D, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(V, D, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g, device="cuda")
    t[:410] = IGN
    return h, w, t


@pytest.mark.parametrize("trainable", [False, True])
def test_planner_matches_measured_loss_peaks(trainable, monkeypatch):
    from mlx_train_perf.core import loss as L
    from mlx_train_perf.plan import estimate as est

    print(f"[planner vs measured peaks, C2, trainable={trainable}]", flush=True)
    monkeypatch.delenv("MTP_LCE_TRANSPOSED_HEAD", raising=False)
    monkeypatch.delenv("MTP_LCE_BWD_BUDGET", raising=False)
    h, w, t = _inputs()
    wd = w.clone().requires_grad_(trainable)
    head = L.DenseHead(weight=wd, trainable=trainable)
    ct = torch.where(t == IGN, 0.0, 1.0 / 8192).float()
    plan = est.loss_bytes(n=N, d=D, v=V, trainable=trainable)
    dh_bytes = N * D * 2
    L.clear_transposed_head_cache()
    torch.cuda.empty_cache()

    def step():
        hd = h.clone().requires_grad_(True)
        fwd, (nll, _, _) = _peak(lambda: L.kernel_forward_parts(hd, head, t, ignore_index=IGN))
        bwd, _ = _peak(lambda: nll.backward(ct))
        wd.grad = None
        return fwd, bwd

    fwd0, bwd0 = step()          # first backward: builds the transposed head
    fwd1, bwd1 = step()          # later steps: the copy is cached
    print(f"  forward {fwd1} B (plan {plan.forward_peak}); backward {bwd1} B (plan {plan.backward_peak} + dH "
          f"{dh_bytes}); first backward {bwd0} B (transposed head {plan.transposed_head})", flush=True)
    assert fwd0 == fwd1 == plan.forward_peak
    # the cotangent the planner counts (n fp32) is the caller's here; autograd adds at most two more.
    # torch's caching allocator may hand each large request (workspace, dH, dW) a whole segment,
    # rounded to 2 MiB, when the remainder is too small to split: up to 2 MiB more per block.
    lo = plan.backward_peak + dh_bytes - N * 4
    assert lo <= bwd1 <= lo + 3 * N * 4 + 3 * (2 << 20), (bwd1, lo)
    assert bwd0 - bwd1 == plan.transposed_head == L.transposed_head_cache_bytes()
    L.clear_transposed_head_cache()


def test_planner_matches_measured_staged_q4_peaks(monkeypatch):
    """A 4-bit head (C3) with the default staged forward and backward: no cached copy; the forward's
    peak is its outputs and the planned workspace (partials, the dequantized head's vocab splits),
    the backward's the planned workspace (gradient tiles, fp32 dH accumulator, one staged head chunk
    and its dequantized rows) and dH."""
    from mlx_train_perf.core import loss as L
    from mlx_train_perf.plan import estimate as est
    from oracle import quant as oquant

    print("[planner vs measured peaks, C3 staged]", flush=True)
    monkeypatch.delenv("MTP_LCE_TRANSPOSED_HEAD", raising=False)
    monkeypatch.delenv("MTP_LCE_STAGE_HEAD", raising=False)
    monkeypatch.delenv("MTP_LCE_BWD_BUDGET", raising=False)
    h, w, t = _inputs()
    wq, sc, bi = (x.cuda() for x in oquant.quantize_affine(w.float(), scale_dtype=torch.bfloat16))
    del w
    head = L.QuantizedHead(w_q=wq, scales=sc, biases=bi)
    ct = torch.where(t == IGN, 0.0, 1.0 / 8192).float()
    plan = est.loss_bytes(n=N, d=D, v=V, quantized=True)
    assert plan.transposed_head == 0
    dh_bytes = N * D * 2
    L.clear_transposed_head_cache()
    torch.cuda.empty_cache()
    peaks = []
    for _ in range(2):
        hd = h.clone().requires_grad_(True)
        fwd, (nll, _, _) = _peak(lambda: L.kernel_forward_parts(hd, head, t, ignore_index=IGN))
        bwd, _ = _peak(lambda: nll.backward(ct))
        peaks.append((fwd, bwd))
    print(f"  forward {peaks[1][0]} B (plan {plan.forward_peak}); backward {peaks[1][1]} B (plan "
          f"{plan.backward_peak} + dH {dh_bytes})", flush=True)
    # the forward's staging workspace (the whole dequantized head here) is one allocation, which the
    # caching allocator rounds up to a multiple of 2 MiB
    assert peaks[0][0] == peaks[1][0]
    assert plan.forward_peak <= peaks[1][0] < plan.forward_peak + (2 << 20)
    lo = plan.backward_peak + dh_bytes - N * 4
    assert lo <= peaks[1][1] <= lo + 3 * N * 4 + 3 * (2 << 20), (peaks[1][1], lo)
    assert abs(peaks[0][1] - peaks[1][1]) <= 2 << 20 and L.transposed_head_cache_bytes() == 0
