"""GPU: mtp_lce_fwd_noalloc (the forward with the library's fixed device scratch instead of a caller
workspace) against mtp_lce_fwd, through the C-ABI: bitwise equal outputs on two calls in a row, the
second smaller than the first (the scratch keeps the first call's partials, which the second must
not read), for a dense and a 4-bit head; a size beyond the scratch is refused before any launch."""
from __future__ import annotations

import pytest
import torch

from oracle import quant as oquant
from tests._inputs import lce_inputs

pytestmark = pytest.mark.gpu

IGN = -100


def _head_args(head: str, w: torch.Tensor):
    from mlx_train_perf import _native

    if head == "dense":
        wd = w.cuda()
        return _native.HEAD_DENSE, (wd.data_ptr(), None, None, None), (wd,)
    wq, sc, bi = (x.cuda() for x in oquant.quantize_affine(w.float(), scale_dtype=torch.bfloat16))
    return _native.HEAD_Q4, (None, wq.data_ptr(), sc.data_ptr(), bi.data_ptr()), (wq, sc, bi)


def _both(n: int, d: int, v: int, head: str, seed: int):
    """(outputs of mtp_lce_fwd, outputs of mtp_lce_fwd_noalloc) for one seeded problem."""
    from mlx_train_perf import _native

    lib = _native.load()
    h, w, t = lce_inputs(n, d, v, seed=seed, ignore_frac=0.1)
    hd, td = h.cuda(), t.cuda()
    kind, ptrs, keep = _head_args(head, w)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for noalloc in (False, True):
        o = [torch.full((n,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(3)]
        if noalloc:
            rc = lib.mtp_lce_fwd_noalloc(hd.data_ptr(), *ptrs, td.data_ptr(), n, d, v, kind, IGN,
                                         o[0].data_ptr(), o[1].data_ptr(), o[2].data_ptr(), stream)
        else:
            ws_b = lib.mtp_lce_fwd_workspace_bytes(n, d, v, kind)
            ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
            rc = lib.mtp_lce_fwd(hd.data_ptr(), *ptrs, td.data_ptr(), n, d, v, kind, IGN, o[0].data_ptr(),
                                 o[1].data_ptr(), o[2].data_ptr(), ws.data_ptr(), ws_b, stream)
        _native.check(rc, domain="loss")
        torch.cuda.synchronize()
        outs.append([x.cpu() for x in o])
    del keep
    return outs


@pytest.mark.parametrize("head", ["dense", "q4"])
def test_noalloc_forward_matches_workspace_forward(head):
    from mlx_train_perf import _native

    lib = _native.load()
    cap = lib.mtp_lce_fwd_noalloc_max_workspace_bytes()
    assert cap == 4 << 20
    # two calls in a row, the second with a smaller problem (fewer tokens and vocab splits)
    for n, d, v, seed in ((2048, 256, 9000, 1), (300, 128, 1027, 2)):
        print(f"[noalloc] head={head} n={n} d={d} v={v}", flush=True)
        assert lib.mtp_lce_fwd_workspace_bytes(n, d, v, 0) <= cap
        ref, got = _both(n, d, v, head, seed)
        for a, b in zip(ref, got):
            assert torch.isfinite(b).all()
            assert torch.equal(a, b)


def test_noalloc_refuses_sizes_beyond_its_scratch():
    from mlx_train_perf import _native
    from mlx_train_perf.errors import LaunchBudgetError

    lib = _native.load()
    cap = lib.mtp_lce_fwd_noalloc_max_workspace_bytes()
    n, d, v = 1 << 20, 64, 4096       # one split x 2^20 tokens x 8 B = 8 MiB of partials
    need = lib.mtp_lce_fwd_workspace_bytes(n, d, v, 0)
    assert need > cap
    print(f"[noalloc] refusal n={n} needs {need} > {cap}", flush=True)
    h = torch.zeros(n, d, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(v, d, dtype=torch.bfloat16, device="cuda")
    t = torch.zeros(n, dtype=torch.int64, device="cuda")
    outs = [torch.full((n,), -1.0, device="cuda") for _ in range(3)]
    rc = lib.mtp_lce_fwd_noalloc(h.data_ptr(), w.data_ptr(), None, None, None, t.data_ptr(), n, d, v, 0, IGN,
                                 outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(),
                                 torch.cuda.current_stream().cuda_stream)
    with pytest.raises(LaunchBudgetError, match="noalloc"):
        _native.check(rc, domain="loss")
    torch.cuda.synchronize()
    assert all(bool((o == -1.0).all()) for o in outs)   # refused before any launch
