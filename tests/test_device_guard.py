"""CPU: every C-ABI call of the product runs with its tensors' device current.

The library launches on the stream it is handed, but some of its HIP calls act on the calling
thread's current device (the no-allocation forward's per-device scratch lookup, error queries), so
the Python layer enters `torch.cuda.device(tensor.device)` around each call. Here `torch.cuda.device`
is replaced by a recorder whose "current device" starts elsewhere, and the library by a stand-in that
records the current device at every entry point the autograd Functions call."""
from __future__ import annotations

import contextlib

import pytest
import torch

from mlx_train_perf import _native
from mlx_train_perf.attention import api as attn_api
from mlx_train_perf.core import loss as L


class _FakeLib:
    def __init__(self, state: dict):
        self.state = state
        self.calls: list[tuple[str, object]] = []

    def _rec(self, name):
        self.calls.append((name, self.state["dev"]))
        return 0

    # attention
    def mtp_attn_fwd(self, *a):
        return self._rec("mtp_attn_fwd")

    def mtp_attn_bwd_workspace_bytes(self, *a):
        return 64

    def mtp_attn_bwd(self, *a):
        return self._rec("mtp_attn_bwd")

    # loss
    def mtp_lce_fwd_workspace_bytes(self, *a):
        return 64

    def mtp_lce_fwd(self, *a):
        return self._rec("mtp_lce_fwd")

    def mtp_lce_bwd_row_block(self, n, *a):
        return n

    def mtp_lce_bwd_chunk(self, n, d, v, budget):
        return 256

    def mtp_lce_bwd_workspace_bytes(self, *a):
        return 64

    def mtp_lce_head_t_ld(self, v):
        return 320

    def mtp_lce_head_transpose(self, *a):
        return self._rec("mtp_lce_head_transpose")

    def mtp_lce_bwd(self, *a):
        return self._rec("mtp_lce_bwd")


@pytest.fixture
def fake(monkeypatch):
    state = {"dev": "cuda:7"}   # the caller's current device is not the tensors'
    lib = _FakeLib(state)

    @contextlib.contextmanager
    def device(dev):
        prev = state["dev"]
        state["dev"] = torch.device(dev)
        try:
            yield
        finally:
            state["dev"] = prev

    monkeypatch.setattr(torch.cuda, "device", device)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(_native, "load", lambda: lib)
    monkeypatch.setattr(_native, "stream_of", lambda t: 0)
    return lib


def test_attention_calls_run_on_the_tensors_device(fake):
    q = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16)
    o, lse = attn_api.kernel_forward(q, k, k, scale=0.125)
    attn_api.kernel_backward(q, k, k, o, lse, torch.zeros_like(q), scale=0.125)
    assert [c[0] for c in fake.calls] == ["mtp_attn_fwd", "mtp_attn_bwd"]
    assert all(dev == q.device for _, dev in fake.calls), fake.calls


def test_loss_calls_run_on_the_tensors_device(fake, monkeypatch):
    monkeypatch.setenv("MTP_LCE_TRANSPOSED_HEAD", "1")
    L.clear_transposed_head_cache()
    n, d, v = 4, 64, 300
    h = torch.zeros(n, d, dtype=torch.bfloat16, requires_grad=True)
    w = torch.zeros(v, d, dtype=torch.bfloat16)
    t = torch.zeros(n, dtype=torch.int64)
    nll, _, _ = L._KernelLCE.apply(h, t, w, None, None, None, _native.HEAD_DENSE, -100, 0, w)
    nll.sum().backward()
    L.clear_transposed_head_cache()
    assert [c[0] for c in fake.calls] == ["mtp_lce_fwd", "mtp_lce_head_transpose", "mtp_lce_bwd"]
    assert all(dev == h.device for _, dev in fake.calls), fake.calls


def test_recorder_sees_a_missing_guard(fake):
    """The recorder would catch a call made outside the guard (the current device stays cuda:7)."""
    fake.mtp_attn_fwd()
    assert fake.calls[-1][1] == "cuda:7"
