"""Launch/memory planner math (CPU): exact causal pair counts by brute force (reference
tests/test_attention_launch_plan.py:61), packed pair counts, LCE split/chunk invariants."""
from __future__ import annotations

import pytest

from mlx_train_perf.plan import launch as plan


@pytest.mark.parametrize("n", [1, 2, 3, 31, 64, 257])
def test_causal_pairs_brute_force(n):
    assert plan.causal_pairs(n) == sum(1 for i in range(n) for j in range(n) if j <= i)


def test_flagship_pair_count():
    assert plan.causal_pairs(8192) == 33_558_528
    flops = 2 * 7 * 128 * 32 * plan.causal_pairs(8192)
    assert abs(flops / 1e12 - 1.924) < 1e-3


def test_packed_pairs_sum_of_segments():
    assert plan.packed_pairs([3, 5]) == 6 + 15
    assert plan.packed_pairs([8]) == plan.causal_pairs(8)


@pytest.mark.parametrize(("n", "v"), [(8192, 151936), (1024, 32000), (65, 1027), (1, 1), (300, 300)])
def test_lce_forward_splits(n, v):
    ns = plan.lce_fwd_splits(n, v)
    vt = -(-v // 256)
    rt = -(-n // 256)
    assert 1 <= ns <= vt
    if vt >= 256:
        assert rt * ns >= 256  # at least one workgroup per CU
    assert plan.lce_fwd_workspace_bytes(n, v) == 8 * ns * n


def test_lce_splits_fill_whole_rounds():
    """Persistent-launch splits: a split count that just overflows one resident round (48 row tiles x
    6 splits = 288 workgroups on 256 CUs) is never chosen; the makespan (rounds x tiles per split)
    stays within 5% of the rule "about one workgroup per CU, rounded up to a multiple of 8" (the plan
    takes the fewest splits within 5% of its cheapest count) and is often far below it."""
    def makespan(rt, vt, ns):
        return -(-(rt * ns) // 256) * -(-vt // ns)

    assert plan.lce_fwd_splits(8192, 151936) == 8           # one round of 32 x 8, the flagship
    # XCD rectangles (256 / ns row tiles x ns splits per round) when within 5% of the cheapest count
    assert plan.lce_fwd_splits(12288, 32000) == 16         # 3 rounds of 16 x 16, not 2 rounds of 48 x 6
    assert plan.lce_fwd_splits(12288, 151936) == 16
    assert plan.lce_fwd_splits(16384, 128256) == 8         # 2 rounds of 32 x 8
    assert plan.lce_fwd_splits(65536, 151936) == 8         # 8 rounds of 32 x 8, not 1 split per row tile
    assert plan.lce_fwd_splits(30720, 151936) == 2         # 120 row tiles: no rectangle; fewest splits
    for n in (256, 1000, 2048, 4096, 8192, 12288, 16384, 65536):
        for v in (1024, 32000, 128256, 151936, 262144):
            rt, vt = -(-n // 256), -(-v // 256)
            ns = plan.lce_fwd_splits(n, v)
            old = -(-256 // rt)
            old = min(-(-old // 8) * 8 if old >= 8 else old, vt)
            assert makespan(rt, vt, ns) <= 1.05 * makespan(rt, vt, max(old, 1)) + 1, (n, v)


def test_lce_forward_partials_fit_the_noalloc_scratch():
    """At most 2048 forward workgroups, so splits x n <= 524288 and the partials [2][splits][n] fp32
    fit the 4 MiB no-alloc scratch for every n <= 524288, whatever v."""
    for v in (1, 1000, 32000, 151936, 262144, 1 << 20):
        for n in list(range(256, 70000, 256)) + [131072, 300000, 524288]:
            assert plan.lce_fwd_workspace_bytes(n, v) <= 4 << 20, (n, v)
    assert plan.lce_fwd_workspace_bytes(524289, 151936) > 4 << 20


def test_lce_dh_split_fills_rounds():
    """The dH contraction is split only when its output tiles leave the last resident round part
    empty: 16 x 16 tiles (the flagship's 4096-row blocks) and any multiple of 256 tiles stay whole;
    16 x 20 tiles (D = 5120) take 4 parts (5 rounds of a quarter of the vocab instead of 2 whole
    rounds), 8 x 16 (N = 2048) take 2; parts never exceed 8 or leave fewer than 8 k tiles each."""
    assert plan.lce_dh_ksplit(4096, 4096, 594) == 1
    assert plan.lce_dh_ksplit(8192, 8192, 594) == 1
    assert plan.lce_dh_ksplit(4096, 5120, 594) == 4
    assert plan.lce_dh_ksplit(2048, 4096, 594) == 2
    assert plan.lce_dh_ksplit(8192, 896, 594) == 2
    assert plan.lce_dh_ksplit(64, 64, 15) == 1
    for rows in (256, 1000, 4096, 8192):
        for d in (64, 896, 2048, 4096, 5120):
            for kt in (1, 7, 16, 100, 594):
                ks = plan.lce_dh_ksplit(rows, d, kt)
                assert 1 <= ks <= 8 and (ks == 1 or kt >= 8 * ks)
                tiles = -(-rows // 256) * -(-d // 256)
                # a split never adds resident rounds of whole-vocab work
                assert -(-(tiles * ks) // 256) * -(-kt // ks) <= -(-tiles // 256) * kt
    # the workspace adds the fp32 part tiles only when the product is split
    assert plan.lce_dh_parts_bytes(4096, 4096, 594) == 0
    assert plan.lce_dh_parts_bytes(4096, 5120, 594) == 4 * 320 * 256 * 256 * 4


def test_flagship_forward_workspace_under_10mb():
    p = plan.lce_plan(n=8192, v=151936, d=4096)
    assert p.fwd_workspace_bytes + 3 * 8192 * 4 < 0.01e9
    assert p.fwd_splits == 8  # 32 row tiles x 8 splits = 1 workgroup per CU


@pytest.mark.parametrize("budget", [1 << 20, 1 << 28, 1 << 30, 1 << 33])
def test_backward_chunk_fits_budget_when_possible(budget):
    n, d, v = 8192, 4096, 151936
    c = plan.lce_bwd_chunk(n, d, v, budget)
    ws = plan.lce_bwd_workspace_bytes(n, d, v, c)
    assert c % 256 == 0
    if c > 256:
        assert ws <= budget
    if budget >= n * (-(-v // 256) * 256 + plan.G_PITCH_PAD) * 2:
        # one chunk: only the bf16 gradient tiles (row pitch padded by 64 elements), no fp32 dH
        assert -(-v // c) == 1 and ws == n * (c + 64) * 2


def test_backward_row_blocks():
    """The default budget (1.5 GiB) runs the flagship backward as two row blocks of one whole-vocab
    chunk each: G holds half the (N, V) gradient, there is no fp32 dH accumulator, and each block's
    dH product still has one 256 x 256 output tile per CU. A trainable head keeps one block."""
    n, d, v = 8192, 4096, 151936
    p = plan.lce_plan(n=n, v=v, d=d)
    assert plan.DEFAULT_LCE_BWD_BUDGET == 3 << 29
    assert (p.bwd_row_block, p.bwd_row_blocks, p.bwd_chunks) == (4096, 2, 1)
    assert p.bwd_workspace_bytes == 4096 * (152064 + 64) * 2 <= plan.DEFAULT_LCE_BWD_BUDGET
    assert (4096 // 256) * (4096 // 256) >= plan.NUM_CU
    t = plan.lce_plan(n=n, v=v, d=d, trainable=True)
    assert t.bwd_row_block == n and t.bwd_chunks > 1 and t.bwd_workspace_bytes <= plan.DEFAULT_LCE_BWD_BUDGET
    # row blocks never leave fewer dH tiles than CUs: at d=1024 the flagship falls back to vocab chunks
    assert plan.lce_bwd_row_block(n, 1024, v, 3 << 29) == n
    # every block but the last is whole; blocks cover the rows
    for nn in (8192, 8200, 12000):
        rb = plan.lce_bwd_row_block(nn, d, v, 3 << 29)
        assert rb % 256 == 0 or rb == nn
        assert -(-nn // rb) * rb >= nn


def test_attention_plan():
    p = plan.attn_plan(b=1, hq=32, hkv=8, s=8192)
    assert p.heads_per_workgroup == 4
    assert p.fwd_workgroups == (8192 // 32) * 8
    assert p.dkv_splits == 1 and p.dkv_workgroups == 64 * 8
    # D, no split at the flagship, the packed work orders (256 query blocks, 64 key blocks), the
    # packed segment ends (one per position)
    assert p.bwd_workspace_bytes == 32 * 8192 * 4 + 256 * 4 + 256 + 8192 * 4
    assert plan.attn_heads_per_workgroup(6, 3) == 2 and plan.attn_heads_per_workgroup(3, 1) == 1


def _dkv_items(b, hq, hkv, s, causal):
    """Brute force: the (head, 64-query tile) items each 128-key block of the dK/dV pass visits."""
    g = hq // hkv
    blocks = []
    for kb in range(-(-s // 128)):
        tiles = [t for t in range(-(-s // 64)) if not causal or (t + 1) * 64 - 1 >= kb * 128]
        blocks.append(g * len(tiles))
    return [x for x in blocks for _ in range(b * hkv)]


@pytest.mark.parametrize("causal", [True, False])
def test_dkv_split_table(causal):
    """The dK/dV size table: known entries at B=1, Hq=32, Hkv=8 (8 splits at S<=1024, 4 at 2048, 2 at
    4096, 1 from 8192), and for every shape the chosen count is the smallest of 1/2/4/8 that brings the
    heaviest workgroup (brute-force item counts) to <= 1.15x a CU's share, the split work adds up to
    the unsplit work, and the workspace holds D plus the partials."""
    if causal:
        assert [plan.attn_dkv_splits(b=1, hq=32, hkv=8, s=s) for s in (512, 1024, 2048, 4096, 8192, 16384)] == \
            [8, 8, 4, 2, 1, 1]
    for b, hq, hkv, s in [(1, 32, 8, 2048), (1, 32, 8, 4096), (2, 32, 8, 2048), (4, 32, 8, 2048), (1, 8, 2, 300),
                          (1, 4, 1, 1100), (1, 32, 8, 8192), (1, 64, 8, 3000), (3, 16, 4, 777)]:
        items = _dkv_items(b, hq, hkv, s, causal)
        share = sum(items) / plan.NUM_CU
        ns = plan.attn_dkv_splits(b=b, hq=hq, hkv=hkv, s=s, causal=causal)
        assert ns in (1, 2, 4, 8)
        fits = [k for k in (1, 2, 4, 8) if max(items) / k <= 1.15 * share]
        assert ns == (fits[0] if fits else 8), (b, hq, hkv, s, ns)
        # the kernel's split of a block of n items: [n * i // ns, n * (i + 1) // ns) for i < ns
        for n in set(items):
            parts = [n * (i + 1) // ns - n * i // ns for i in range(ns)]
            assert sum(parts) == n and max(parts) - min(parts) <= 1
    assert plan.attn_dkv_splits(b=1, hq=32, hkv=8, s=2048, dh=64) == 4   # the same table for head_dim 64/96
    ws = plan.attn_bwd_workspace_bytes(b=1, hq=32, hkv=8, s=2048)
    # D, 4 splits of fp32 dK and dV, then the packed work orders: 64 query blocks of 32 and 16 key
    # blocks of 128, an int32 each, each order padded to 256 bytes, and an int32 segment end per
    # position
    assert ws == 32 * 2048 * 4 + 4 * 2 * 8 * 2048 * 128 * 4 + 256 + 256 + 2048 * 4
    # D padded to 256 bytes before the partials (their 16-byte stores stay aligned); one head per
    # workgroup gives 128-query blocks
    assert plan.attn_bwd_workspace_bytes(b=1, hq=1, hkv=1, s=61) == 256 + 8 * 2 * 61 * 128 * 4 + 256 + 256 + 256


def test_memory_planner_terms():
    from mlx_train_perf.errors import DoesNotFitError, PlanInputError
    from mlx_train_perf.plan import estimate as est

    lb = est.loss_bytes(n=8192, d=4096, v=151936, impl="kernel")
    assert lb.forward_peak == 3 * 8192 * 4 + plan.lce_fwd_workspace_bytes(8192, 151936) < 0.01e9
    assert est.loss_bytes(n=8192, d=4096, v=151936, impl="naive").forward_peak > 4.9e9
    assert est.flash_saved_state_bytes(batch=1, seq_len=8192, heads=32, head_dim=128) == 8192 * 32 * 128 * 2 + 8192 * 32 * 4
    p = est.estimate_peak(n_layers=32, batch=1, seq_len=8192, hidden=4096, vocab=151936, heads=32, kv_heads=8,
                          head_dim=128, weights_bytes=16 * 10**9)
    assert est.plan_fit(p, budget_bytes=288 * 10**9) == p.total
    with pytest.raises(DoesNotFitError):
        est.plan_fit(p, budget_bytes=10 * 10**9)
    stock = est.estimate_peak(n_layers=32, batch=1, seq_len=8192, hidden=4096, vocab=151936, heads=32, kv_heads=8,
                              head_dim=128, attention="stock", loss_impl="naive")
    assert stock.components["attention"] > p.components["attention"]
    with pytest.raises(PlanInputError):
        est.loss_bytes(n=1, d=1, v=1, impl="fast")


def test_memory_planner_head_terms():
    """The cached transposed head and a trainable head's dL/dW (and its all-rows backward block)."""
    from mlx_train_perf.plan import estimate as est

    n, d, v = 8192, 4096, 151936
    frozen = est.loss_bytes(n=n, d=d, v=v, transposed_head=True)
    # [d][round_up(v, 256) + 64] bf16 = 1.246 GB, the copy the backward reads for its dH product
    assert frozen.transposed_head == d * (152064 + 64) * 2 == 1_246_232_576
    assert est.loss_bytes(n=n, d=d, v=v, transposed_head=False).transposed_head == 0
    assert est.loss_bytes(n=n, d=100, v=v, transposed_head=True).transposed_head == 0   # d % 64: no copy
    assert frozen.head_grad == 0 and frozen.peak == frozen.transposed_head + frozen.backward_workspace
    # frozen flagship: two 4096-row blocks of one vocab chunk (1.25 GB of gradient tiles)
    assert frozen.backward_workspace == 4096 * (152064 + 64) * 2 + n * 4
    # a trainable head without the copy: every row in one block, each vocab chunk of the head staged
    # in the workspace (3 chunks of 59904 columns within the 1.5 GiB budget)
    tr = est.loss_bytes(n=n, d=d, v=v, trainable=True, transposed_head=False)
    p = plan.lce_plan(n=n, v=v, d=d, trainable=True, staged=True)
    assert p.bwd_row_block == n and p.bwd_chunk == 59904 and p.bwd_chunks == 3
    assert tr.head_grad == v * d * 2 and tr.backward_workspace == p.bwd_workspace_bytes + n * 4
    # and with it (two chunks of gradient tiles, no staging buffer)
    trc = est.loss_bytes(n=n, d=d, v=v, trainable=True, transposed_head=True)
    pc = plan.lce_plan(n=n, v=v, d=d, trainable=True)
    assert pc.bwd_row_block == n and pc.bwd_chunks == 2
    assert trc.backward_workspace == pc.bwd_workspace_bytes + n * 4
    assert tr.backward_peak == tr.backward_workspace + tr.head_grad > 2.8e9
    step = dict(n_layers=32, batch=1, seq_len=8192, hidden=d, vocab=v, heads=32, kv_heads=8, head_dim=128)
    full = est.estimate_peak(**step, trainable_head=True).components["loss"]
    lora = est.estimate_peak(**step).components["loss"]
    # by default a frozen dense head keeps the transposed copy and a trainable one stages its chunks
    full_lb, lora_lb = est.loss_bytes(n=n, d=d, v=v, trainable=True), est.loss_bytes(n=n, d=d, v=v)
    assert full == full_lb.peak and lora == lora_lb.peak
    assert full_lb.head_grad == v * d * 2 and full_lb.transposed_head == 0 < lora_lb.transposed_head
    assert full_lb.backward_peak > lora_lb.backward_peak + v * d * 2
    # the chunked and naive impls carry the dL/dW term too
    assert est.loss_bytes(n=n, d=d, v=v, impl="chunked", trainable=True).head_grad == v * d * 2


def test_memory_planner_quantized_head_staging(monkeypatch):
    """A 4-bit head (QLoRA, config 3): the backward stages each vocab chunk's dequantized rows and the
    chunk transposed (4 chunks of 44800 columns within 1.5 GiB: 2N + 4D bytes per column); the bf16
    forward stages the whole dequantized head when it fits the budget (one launch over every vocab
    split), else it dequantizes in registers with only the split partials; MTP_LCE_STAGE_HEAD=0
    stages nothing."""
    from mlx_train_perf.plan import estimate as est

    monkeypatch.delenv("MTP_LCE_STAGE_HEAD", raising=False)
    monkeypatch.delenv("MTP_LCE_TRANSPOSED_HEAD", raising=False)
    n, d, v = 8192, 4096, 151936
    budget = 3 << 29
    p = plan.lce_plan(n=n, v=v, d=d, budget=budget, staged=True, quantized=True, fwd_staged=True)
    assert p.bwd_row_block == n and p.bwd_chunk == 44800 and p.bwd_chunks == 4
    partials = plan.lce_fwd_workspace_bytes(n, v)
    whole = -(-partials // 256) * 256 + v * d * 2
    assert plan.lce_fwd_stages_whole_head(n, d, v, budget) and p.fwd_workspace_bytes == whole
    q = est.loss_bytes(n=n, d=d, v=v, quantized=True, bwd_budget=budget)
    assert q.transposed_head == 0
    assert q.forward_peak == 3 * n * 4 + whole < q.backward_workspace
    assert q.backward_workspace == p.bwd_workspace_bytes + n * 4
    # a budget below the whole head: the forward dequantizes in registers
    small = 3 << 28
    assert not plan.lce_fwd_stages_whole_head(n, d, v, small)
    assert est.loss_bytes(n=n, d=d, v=v, quantized=True, bwd_budget=small).forward_peak == 3 * n * 4 + partials
    # fp32 inputs and d % 64 != 0 never stage the forward
    assert est.loss_bytes(n=n, d=d, v=v, quantized=True, dtype="fp32", bwd_budget=budget).forward_peak == 3 * n * 4 + partials
    assert not plan.lce_fwd_stages_whole_head(n, 4000, v, 1 << 40)
    monkeypatch.setenv("MTP_LCE_STAGE_HEAD", "0")
    assert est.loss_bytes(n=n, d=d, v=v, quantized=True, bwd_budget=budget).forward_peak == 3 * n * 4 + partials
