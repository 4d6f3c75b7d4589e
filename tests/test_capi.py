"""The C-ABI library (CPU lane): it loads, exports every symbol the headers declare, reports the
same plans as the Python planner, and refuses invalid calls with typed codes before any launch.
No call here reaches a GPU launch: every case fails validation or is a pure size query."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from mlx_train_perf import _native
from mlx_train_perf.plan import launch as plan

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        names |= set(re.findall(r"\b(mtp_\w+)\s*\(", h.read_text()))
    return names


@pytest.mark.parametrize("kind", ["q4", "dense"])
@pytest.mark.parametrize("budget", [3 << 29, 3 << 28, 1 << 28, 1 << 30, 1 << 20])
@pytest.mark.parametrize(("n", "d", "v"), [(8192, 4096, 151936), (1024, 512, 32000), (65, 192, 1027),
                                           (2048, 4096, 151936), (1000, 2048, 8000), (16384, 8192, 262144)])
def test_staged_plan_agrees_with_python_planner(n, d, v, budget, kind):
    """The staged backward's chunk and workspace (gradient tiles, accumulator, part tiles, then the
    staging buffer: the transposed chunk, and for a 4-bit head its dequantized rows) agree between
    the library and plan/launch.py, and fit the budget's terms."""
    from mlx_train_perf import _native as N

    q4 = kind == "q4"
    hk = N.HEAD_Q4_STAGED if q4 else N.HEAD_DENSE_STAGED
    lib = _native.load()
    assert lib.mtp_lce_bwd_stage_chunk(n, d, v, N.HEAD_Q4, budget) == 0   # not a staged kind
    c = lib.mtp_lce_bwd_stage_chunk(n, d, v, hk, budget)
    assert c == plan.lce_stage_chunk(n, d, v, budget, quantized=q4)
    assert c % 256 == 0 and 256 <= c <= (v + 255) // 256 * 256
    ws = lib.mtp_lce_bwd_workspace_bytes(n, d, v, hk, c, n)
    assert ws == plan.lce_bwd_workspace_bytes(n, d, v, c, n, staged=True, quantized=q4)
    plain = lib.mtp_lce_bwd_workspace_bytes(n, d, v, N.HEAD_Q4, c, n)
    stage = d * lib.mtp_lce_head_t_ld(c) * 2
    if q4:   # the rows follow the transposed chunk at a 256-byte boundary
        stage = -(-stage // 256) * 256 + c * d * 2
    assert ws == -(-plain // 256) * 256 + stage
    if c > 256:   # a chunk above the minimum fits the budget (the part tiles are outside it)
        nchunks = -(-v // c)
        per_col = 2 * (n + d) + (2 * d if q4 else 0)
        assert per_col * (c + 64) + (n * d * 4 if nchunks > 1 else 0) <= budget


@pytest.mark.parametrize("budget", [3 << 29, 1 << 28, 1 << 24, 0, 1 << 40])
@pytest.mark.parametrize(("n", "d", "v"), [(8192, 4096, 151936), (4096, 4096, 151936), (1000, 512, 20000),
                                           (513, 192, 7777), (64, 64, 1000), (2048, 1024, 40000), (100, 96, 500),
                                           (256, 128, 262144), (512, 64, 200000)])
def test_staged_forward_workspace_agrees_with_python_planner(n, d, v, budget):
    """The staged 4-bit forward's workspace (partials, then the largest run of whole vocab splits
    whose rows fit the budget) agrees between the library and plan/launch.py; the least it takes is
    one split's rows, the most the whole head's; d not a multiple of 64 stages nothing."""
    from mlx_train_perf import _native as N

    lib = _native.load()
    ws = lib.mtp_lce_fwd_stage_workspace_bytes(n, d, v, budget)
    if d % 64:
        assert ws == 0 == plan.lce_fwd_stage_workspace_bytes(n, d, v, budget)
        return
    assert ws == plan.lce_fwd_stage_workspace_bytes(n, d, v, budget)
    off = -(-plan.lce_fwd_workspace_bytes(n, v) // 256) * 256
    ns = plan.lce_fwd_splits(n, v)
    one = max(plan.lce_fwd_split_rows(n, v, s, s + 1, ns) for s in range(ns))
    assert lib.mtp_lce_fwd_workspace_bytes(n, d, v, N.HEAD_Q4_STAGED) == off + one * d * 2
    assert off + one * d * 2 <= ws <= off + v * d * 2
    assert sum(plan.lce_fwd_split_rows(n, v, s, s + 1, ns) for s in range(ns)) == v
    if budget >= off + v * d * 2:
        assert ws == off + v * d * 2
    elif ws > off + one * d * 2:
        assert ws <= budget


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    declared = _declared_symbols()
    assert {"mtp_lce_fwd", "mtp_lce_bwd", "mtp_attn_fwd", "mtp_attn_bwd"} <= declared
    for name in declared:
        assert hasattr(lib, name), name
    assert set(_native.SIGNATURES) >= declared - set()  # every export has a Python signature
    assert lib.mtp_abi_version() == _native.ABI_VERSION == 5


@pytest.mark.parametrize(("n", "d", "v"), [(8192, 4096, 151936), (1024, 512, 32000), (65, 192, 1027), (1, 8, 1),
                                           (8192, 5120, 152064), (2048, 4096, 151936), (8192, 1536, 151936),
                                           (12288, 4096, 32000), (4352, 3584, 152064), (1000, 2048, 8000)])
def test_plans_agree_with_python_planner(n, d, v):
    lib = _native.load()
    assert lib.mtp_lce_fwd_workspace_bytes(n, d, v, 0) == plan.lce_fwd_workspace_bytes(n, v)
    for budget in (1 << 20, 1 << 26, 1 << 30, 3 << 29, 1 << 34):
        c = lib.mtp_lce_bwd_chunk(n, d, v, budget)
        assert c == plan.lce_bwd_chunk(n, d, v, budget)
        assert c % 256 == 0 and c >= 256
        rb = lib.mtp_lce_bwd_row_block(n, d, v, budget)
        assert rb == plan.lce_bwd_row_block(n, d, v, budget)
        for rows in (0, n, rb):
            assert lib.mtp_lce_bwd_workspace_bytes(n, d, v, 0, c, rows) == plan.lce_bwd_workspace_bytes(n, d, v, c, rows)
        p = plan.lce_plan(n=n, v=v, d=d, budget=budget)
        assert p.bwd_row_block == rb
        assert p.bwd_workspace_bytes == lib.mtp_lce_bwd_workspace_bytes(n, d, v, 0, p.bwd_chunk, rb)
    assert lib.mtp_attn_bwd_workspace_bytes(1, 32, 8, 8192, 128) == plan.attn_plan(b=1, hq=32, hkv=8, s=8192).bwd_workspace_bytes


@settings(max_examples=400, deadline=None, derandomize=True)
@given(n=st.integers(1, 1 << 17), d=st.integers(1, 160).map(lambda k: 64 * k), v=st.integers(1, 1 << 18),
       budget_log2=st.integers(16, 36))
def test_plans_agree_over_random_shapes(n, d, v, budget_log2):
    """The Python mirrors of the launch planner (vocab splits, chunks, row blocks, dH contraction
    parts, workspace sizes) against the library over seeded random shapes and budgets."""
    lib = _native.load()
    budget = 1 << budget_log2
    assert lib.mtp_lce_fwd_workspace_bytes(n, d, v, 0) == plan.lce_fwd_workspace_bytes(n, v)
    c = lib.mtp_lce_bwd_chunk(n, d, v, budget)
    assert c == plan.lce_bwd_chunk(n, d, v, budget)
    rb = lib.mtp_lce_bwd_row_block(n, d, v, budget)
    assert rb == plan.lce_bwd_row_block(n, d, v, budget)
    # 0, a negative count and one above n all mean every row (capi.hip clamps row_block < 1 to n)
    for rows in (0, -1, -rb, n, n + 1, rb):
        assert lib.mtp_lce_bwd_workspace_bytes(n, d, v, 0, c, rows) == plan.lce_bwd_workspace_bytes(n, d, v, c, rows)


@settings(max_examples=300, deadline=None, derandomize=True)
@given(b=st.integers(1, 8), hkv=st.sampled_from([1, 2, 4, 8]), g=st.sampled_from([1, 2, 3, 4, 8]),
       s=st.integers(1, 40000), dh=st.sampled_from([64, 96, 128]), causal=st.booleans())
def test_attention_plans_agree_over_random_shapes(b, hkv, g, s, dh, causal):
    lib = _native.load()
    hq = hkv * g
    assert lib.mtp_attn_bwd_dkv_splits(b, hq, hkv, s, dh, int(causal)) == plan.attn_dkv_splits(
        b=b, hq=hq, hkv=hkv, s=s, dh=dh, causal=causal)
    assert lib.mtp_attn_bwd_workspace_bytes(b, hq, hkv, s, dh) == plan.attn_bwd_workspace_bytes(
        b=b, hq=hq, hkv=hkv, s=s, dh=dh)


def test_dkv_split_table_agrees_with_python_planner():
    lib = _native.load()
    for b in (1, 2, 4):
        for hq, hkv in ((32, 8), (8, 2), (4, 1), (6, 3), (64, 8)):
            for s in (1, 61, 300, 1024, 1100, 2048, 4096, 5000, 8192, 16384):
                for dh in (64, 96, 128):
                    for causal in (0, 1):
                        assert lib.mtp_attn_bwd_dkv_splits(b, hq, hkv, s, dh, causal) == plan.attn_dkv_splits(
                            b=b, hq=hq, hkv=hkv, s=s, dh=dh, causal=bool(causal)), (b, hq, hkv, s, dh, causal)
                    assert lib.mtp_attn_bwd_workspace_bytes(b, hq, hkv, s, dh) == plan.attn_bwd_workspace_bytes(
                        b=b, hq=hq, hkv=hkv, s=s, dh=dh)


FAKE = 0x100000  # aligned, never dereferenced: every call below fails validation first


def _lce_fwd(**kw):
    lib = _native.load()
    a = dict(hidden=FAKE, w=FAKE, w_q=None, scales=None, biases=None, targets=FAKE, n=16, d=64, v=100, head=0,
             ign=-100, nll=FAKE, lse=FAKE, tgt=FAKE, ws=FAKE, ws_bytes=0, stream=None)
    a.update(kw)
    return lib.mtp_lce_fwd(a["hidden"], a["w"], a["w_q"], a["scales"], a["biases"], a["targets"], a["n"], a["d"],
                           a["v"], a["head"], a["ign"], a["nll"], a["lse"], a["tgt"], a["ws"], a["ws_bytes"], a["stream"])


def test_lce_refusals():
    assert _lce_fwd(n=0) == _native.MTP_ERR_INPUT
    assert _lce_fwd(targets=None) == _native.MTP_ERR_INPUT
    assert _lce_fwd(d=33) == _native.MTP_ERR_UNSUPPORTED
    assert _lce_fwd(hidden=FAKE + 2) == _native.MTP_ERR_UNSUPPORTED
    assert _lce_fwd(head=1, w=None, w_q=FAKE, scales=FAKE, biases=FAKE, d=96) == _native.MTP_ERR_UNSUPPORTED
    assert _lce_fwd(head=7) == _native.MTP_ERR_UNSUPPORTED
    assert _lce_fwd(ws_bytes=8) == _native.MTP_ERR_WORKSPACE
    assert "workspace" in _native.last_error()
    lib = _native.load()
    rc = lib.mtp_lce_bwd(FAKE, FAKE, None, None, None, None, FAKE, 16, 64, 100, 0, -100, FAKE, FAKE, FAKE, None, 100, 0, FAKE, 1 << 20, None)
    assert rc == _native.MTP_ERR_INPUT and "multiple of 256" in _native.last_error()
    rc = lib.mtp_lce_bwd(FAKE, FAKE, None, None, None, None, FAKE, 16, 64, 100, 0, -100, FAKE, FAKE, FAKE, None, 256, 0, FAKE, 16, None)
    assert rc == _native.MTP_ERR_WORKSPACE
    rc = lib.mtp_lce_bwd(FAKE, None, None, FAKE, FAKE, FAKE, FAKE, 16, 64, 100, 1, -100, FAKE, FAKE, FAKE, FAKE, 256, 0, FAKE, 1 << 20, None)
    assert rc == _native.MTP_ERR_UNSUPPORTED and "frozen" in _native.last_error()
    # row blocks: a multiple of 256 below n, and never with a trainable head's d_w
    rc = lib.mtp_lce_bwd(FAKE, FAKE, None, None, None, None, FAKE, 1024, 64, 100, 0, -100, FAKE, FAKE, FAKE, None, 256, 300, FAKE, 1 << 30, None)
    assert rc == _native.MTP_ERR_INPUT and "row_block" in _native.last_error()
    rc = lib.mtp_lce_bwd(FAKE, FAKE, None, None, None, None, FAKE, 1024, 64, 100, 0, -100, FAKE, FAKE, FAKE, FAKE, 256, 512, FAKE, 1 << 30, None)
    assert rc == _native.MTP_ERR_INPUT and "trainable" in _native.last_error()
    assert lib.mtp_lce_head_t_ld(151936) == 152064 + 64 and lib.mtp_lce_head_t_ld(1) == 256 + 64
    assert lib.mtp_lce_head_transpose(FAKE, None, None, None, 100, 36, 0, FAKE, None) == _native.MTP_ERR_UNSUPPORTED
    assert lib.mtp_lce_head_transpose(None, None, None, None, 100, 64, 0, FAKE, None) == _native.MTP_ERR_INPUT
    assert lib.mtp_lce_head_transpose(None, FAKE, FAKE, FAKE, 100, 96, 1, FAKE, None) == _native.MTP_ERR_UNSUPPORTED
    assert lib.mtp_lce_head_transpose(None, FAKE, None, FAKE, 100, 64, 1, FAKE, None) == _native.MTP_ERR_INPUT


def test_attention_refusals():
    lib = _native.load()

    def fwd(**kw):
        a = dict(b=1, hq=4, hkv=2, s=16, dh=64, causal=1, sid=None, sst=None)
        a.update(kw)
        return lib.mtp_attn_fwd(FAKE, FAKE, FAKE, a["b"], a["hq"], a["hkv"], a["s"], a["dh"], 0.1, a["causal"],
                                a["sid"], a["sst"], (FAKE if kw.get("o", True) else None), FAKE, None)

    assert fwd(hq=3) == _native.MTP_ERR_INPUT
    assert fwd(dh=80) == _native.MTP_ERR_UNSUPPORTED
    assert fwd(causal=2) == _native.MTP_ERR_INPUT
    assert fwd(causal=0, sid=FAKE, sst=FAKE) == _native.MTP_ERR_UNSUPPORTED   # packed needs causal
    assert fwd(sid=FAKE) == _native.MTP_ERR_INPUT
    assert fwd(o=False) == _native.MTP_ERR_INPUT
    rc = lib.mtp_attn_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 4, 2, 16, 64, 0.1, 1, None, None, FAKE, FAKE, FAKE,
                          FAKE, 4, None)
    assert rc == _native.MTP_ERR_WORKSPACE


def test_fp32_entry_points_plan_and_refuse():
    """The fp32 entry points: workspace sizes, the backward's chunk plan, and validation before any
    launch (same codes as the bf16 ones; fp32 takes any d for a dense head)."""
    lib = _native.load()
    # forward partials: [2][splits][n] fp32, about two workgroups per CU of 128-token tiles
    assert lib.mtp_lce_fwd_f32_workspace_bytes(1024, 512, 32000, 0) == 2 * 64 * 1024 * 4
    assert lib.mtp_lce_fwd_f32_workspace_bytes(8192, 4096, 151936, 0) == 2 * 8 * 8192 * 4
    assert lib.mtp_lce_fwd_f32_workspace_bytes(0, 512, 32000, 0) == 0
    # backward: one fp32 gradient tile [n][chunk + 4]; the whole padded vocab when it fits the budget
    assert lib.mtp_lce_bwd_f32_chunk(1024, 512, 32000, 3 << 29) == 32000
    # config 1: 8 x 4 output tiles of dH -> 16 contraction parts of fp32 partial dH after the g tile
    assert lib.mtp_lce_bwd_f32_workspace_bytes(1024, 512, 32000, 32000) == 1024 * 32004 * 4 + 16 * 1024 * 512 * 4
    # a large output grid (64 x 32 tiles) keeps one part: no partials
    assert lib.mtp_lce_bwd_f32_workspace_bytes(8192, 4096, 151936, 1024) == 8192 * 1028 * 4
    # a chunk too short for two 512-column parts keeps one part as well
    assert lib.mtp_lce_bwd_f32_workspace_bytes(1024, 512, 32000, 896) == 1024 * 900 * 4
    c = lib.mtp_lce_bwd_f32_chunk(8192, 4096, 151936, 1 << 30)
    assert c % 128 == 0 and 8192 * (c + 4) * 4 <= 1 << 30 < 8192 * (c + 132) * 4
    assert lib.mtp_lce_bwd_f32_chunk(8, 64, 100, 1) == 128    # at least one 128-column tile
    assert lib.mtp_attn_bwd_f32_workspace_bytes(1, 32, 8, 8192, 128) == 32 * 8192 * 4
    fwd = lambda **kw: lib.mtp_lce_fwd_f32(kw.get("h", FAKE), kw.get("w", FAKE), None, None, None, FAKE, 16,
                                           kw.get("d", 36), 100, kw.get("head", 0), -100, FAKE, FAKE, FAKE, FAKE,
                                           kw.get("ws", 0), None)
    assert fwd() == _native.MTP_ERR_WORKSPACE       # d = 36 is fine for fp32; the workspace is missing
    assert fwd(h=FAKE + 4) == _native.MTP_ERR_UNSUPPORTED
    assert fwd(w=None) == _native.MTP_ERR_INPUT
    assert fwd(head=1) == _native.MTP_ERR_INPUT       # quantized head without its tensors
    rc = lib.mtp_lce_bwd_f32(FAKE, FAKE, None, None, None, FAKE, 16, 64, 100, 0, -100, FAKE, FAKE, FAKE, None, 100,
                             FAKE, 1 << 20, None)
    assert rc == _native.MTP_ERR_INPUT and "multiple of 128" in _native.last_error()
    rc = lib.mtp_attn_fwd_f32(FAKE, FAKE, FAKE, 1, 4, 2, 16, 80, 0.1, 1, None, None, FAKE, FAKE, None)
    assert rc == _native.MTP_ERR_UNSUPPORTED
    rc = lib.mtp_attn_bwd_f32(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 4, 2, 16, 64, 0.1, 1, None, None, FAKE, FAKE,
                              FAKE, FAKE, 4, None)
    assert rc == _native.MTP_ERR_WORKSPACE


def test_error_mapping_to_typed_exceptions():
    from mlx_train_perf.errors import LaunchBudgetError, LossInputError, UnsupportedAttentionError

    with pytest.raises(LossInputError):
        _native.check(_native.MTP_ERR_INPUT, domain="loss")
    with pytest.raises(UnsupportedAttentionError):
        _native.check(_native.MTP_ERR_UNSUPPORTED, domain="attention")
    with pytest.raises(LaunchBudgetError):
        _native.check(_native.MTP_ERR_WORKSPACE, domain="loss")
    assert ctypes.c_int(_native.MTP_OK).value == 0
