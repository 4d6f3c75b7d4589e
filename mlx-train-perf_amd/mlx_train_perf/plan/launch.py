"""Launch planning for the LCE and attention kernels (pure integer math, CPU-testable).

The reference plans Metal dispatches against a GPU-watchdog time budget
(core/kernel/launch.py:63-72; attention/kernel/launch.py:160-299). On MI355X there is no display
watchdog on compute queues, so every op is one launch sequence and the planner's job is geometry and
workspace: how many vocab splits the LCE forward uses, how wide a backward vocab chunk may be for a
workspace budget, and the attention grid. The integer formulas here mirror the C-ABI's
(mlx-train-perf_amd/csrc/lce_kernels.hip lce_nsplit, lce_dh_ksplit; capi.hip mtp_lce_bwd_row_block,
mtp_lce_bwd_chunk, mtp_lce_bwd_workspace_bytes; attn_kernels.hip attn_dkv_nsplit) so that plans
can be checked and sized on the CPU; a GPU test asserts they agree with the library.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

NUM_CU = 256        # MI355X compute units (8 XCDs x 32)
TILE = 256          # LCE workgroup tile edge (rows and vocab columns)
ATTN_TILE = 64      # attention key/query tile
# Bytes of backward workspace (bf16 gradient tiles + fp32 dH when the vocab is chunked). 1.5 GiB
# holds the whole padded vocab of a 151936-entry head for half of 8192 tokens (1.25 GB), so the
# flagship backward runs as two row blocks of one vocab chunk each: G never holds the full (N, V)
# matrix, and there is no fp32 dH read-modify-write. MTP_LCE_BWD_BUDGET overrides it.
DEFAULT_LCE_BWD_BUDGET = 3 << 29


# Gradient-tile rows are chunk + 64 elements apart: a pitch that is a multiple of a large power of
# two puts the rows of one operand tile on the same memory channels (csrc/mtp_launch.hpp).
G_PITCH_PAD = 64


def lce_bwd_budget_bytes() -> int:
    return int(os.environ.get("MTP_LCE_BWD_BUDGET", DEFAULT_LCE_BWD_BUDGET))


def causal_pairs(n: int) -> int:
    """Exact (query, key) pairs under a causal mask (attention/kernel/launch.py:160-168)."""
    return n * (n + 1) // 2


def packed_pairs(lengths: list[int]) -> int:
    """Visible pairs of a block-diagonal causal (packed) layout."""
    return sum(causal_pairs(n) for n in lengths)


FWD_WGS_PER_CU = 1  # forward workgroups per CU (csrc/lce_kernels.hip)


def lce_nsplit(n: int, v: int, per_cu: int = FWD_WGS_PER_CU) -> int:
    """Vocab splits of a persistent LCE launch (forward, and the backward's gradient tiles per
    chunk): cost(ns) = resident rounds x (vocab tiles per split + 1). Within 5% of the cheapest count:
    8, 16 or 32 when the XCD rectangles tile it (n's row tiles a multiple of 256 / ns), else the
    fewest splits (every split adds partials to merge); never more than the vocab tiles, 1024, or
    2048 workgroups in all (so splits x n <= 524288: 4 MiB of forward partials)."""
    rtiles = -(-n // TILE)
    vtiles = -(-v // TILE)
    slots = per_cu * NUM_CU
    top = max(1, min(vtiles, 1024, 2048 // rtiles))

    def cost(ns: int) -> int:
        return -(-(rtiles * ns) // slots) * (-(-vtiles // ns) + 1)

    least = min(cost(ns) for ns in range(1, top + 1))
    if per_cu == 1:   # a count the XCD rectangles tile (256 / ns row tiles x ns splits per round) first
        for ns in (8, 16, 32):
            if ns <= top and rtiles % (256 // ns) == 0 and cost(ns) * 100 <= least * 105:
                return ns
    return next(ns for ns in range(1, top + 1) if cost(ns) * 100 <= least * 105)


def lce_fwd_splits(n: int, v: int) -> int:
    """Vocab splits of the forward (lce_nsplit at FWD_WGS_PER_CU workgroups per CU)."""
    return lce_nsplit(n, v, FWD_WGS_PER_CU)


def lce_dh_ksplit(rows: int, d: int, ktiles: int) -> int:
    """Parts of the backward's dH contraction over `ktiles` 256-wide vocab tiles for a block of
    `rows` rows: the count (1..8, each part >= 8 k tiles) minimizing resident rounds x (k tiles per
    part + 1, or + 4 for an fp32 part) + parts x tiles / 128 for the ordered reduction."""
    tiles = -(-rows // TILE) * -(-d // TILE)
    best, best_cost = 1, -(-tiles // NUM_CU) * (ktiles + 1)
    ks = 2
    while ks <= 8 and ks * 8 <= ktiles:
        cost = -(-(tiles * ks) // NUM_CU) * (-(-ktiles // ks) + 4) + ks * tiles // 128
        if cost < best_cost:
            best, best_cost = ks, cost
        ks += 1
    return best


def lce_dh_parts_bytes(rows: int, d: int, ktiles: int) -> int:
    """fp32 part tiles of a split dH product (0 when it is not split)."""
    ks = lce_dh_ksplit(rows, d, ktiles)
    return 0 if ks == 1 else ks * -(-rows // TILE) * -(-d // TILE) * TILE * TILE * 4


def lce_fwd_workspace_bytes(n: int, v: int) -> int:
    return 2 * lce_fwd_splits(n, v) * n * 4


def lce_fwd_split_rows(n: int, v: int, s0: int, s1: int, ns: int | None = None) -> int:
    """Vocab rows of forward splits [s0, s1) (`ns`: the split count, when the caller has it)."""
    ns = lce_fwd_splits(n, v) if ns is None else ns
    vtiles = -(-v // TILE)
    return min(v, s1 * vtiles // ns * TILE) - s0 * vtiles // ns * TILE


def lce_fwd_stage_workspace_bytes(n: int, d: int, v: int, budget: int) -> int:
    """The staged 4-bit forward's workspace within a budget (mirror of
    mtp_lce_fwd_stage_workspace_bytes): the partials, 256-byte aligned, then a bf16 staging buffer of
    the largest run of whole vocab splits whose rows fit the budget's rest (at least one split)."""
    if d % 64:
        return 0
    ns = lce_fwd_splits(n, v)
    off = -(-lce_fwd_workspace_bytes(n, v) // 256) * 256
    cap = max((budget - off) // (2 * d) if budget > off else 0,
              max(lce_fwd_split_rows(n, v, s, s + 1, ns) for s in range(ns)))
    most, s0 = 0, 0
    while s0 < ns:
        s1 = s0 + 1
        while s1 < ns and lce_fwd_split_rows(n, v, s0, s1 + 1, ns) <= cap:
            s1 += 1
        most = max(most, lce_fwd_split_rows(n, v, s0, s1, ns))
        s0 = s1
    return off + most * d * 2


def lce_bwd_row_block(n: int, d: int, v: int, budget: int) -> int:
    """Rows per backward block (mirror of mtp_lce_bwd_row_block): all n when the whole padded
    vocab's gradient tiles fit the budget; else n split in 2 or 4 blocks (a multiple of 256 rows)
    whose whole-vocab tiles fit it while the dH product keeps >= NUM_CU output tiles; else, when
    chunking the vocab would take more than 4 chunks, 8 or 16 blocks that fit (their dH products
    split the contraction); else n."""
    vpad = -(-v // TILE) * TILE
    row_bytes = (vpad + G_PITCH_PAD) * 2
    if n * row_bytes <= budget:
        return n
    for parts in (2, 4):
        rows = -(-(-(-n // parts)) // TILE) * TILE
        if (rows // TILE) * -(-d // TILE) < NUM_CU:
            break
        if rows * row_bytes <= budget:
            return rows
    if -(-v // lce_bwd_chunk(n, d, v, budget)) > 4:
        for parts in (8, 16):
            rows = -(-(-(-n // parts)) // TILE) * TILE
            if rows * row_bytes <= budget:
                return rows
    return n


def lce_bwd_chunk(n: int, d: int, v: int, budget: int) -> int:
    """Vocab columns per backward chunk (multiple of 256) for a workspace budget in bytes."""
    vpad = -(-v // TILE) * TILE
    if n * (vpad + G_PITCH_PAD) * 2 <= budget:
        return vpad
    acc = n * d * 4
    rest = max(budget - acc, 0)
    c = (rest // (n * 2) - G_PITCH_PAD) // TILE * TILE
    return min(max(c, TILE), vpad)


def lce_bwd_workspace_bytes(n: int, d: int, v: int, chunk: int, row_block: int | None = None, *,
                            staged: bool = False, quantized: bool = False) -> int:
    """bf16 gradient tiles [row_block][chunk + G_PITCH_PAD], the fp32 dH accumulator when >1 chunk,
    and the fp32 part tiles of a split dH product (the most any row block and chunk takes); `staged`
    (the MTP_HEAD_*_STAGED backwards): then, 256-byte aligned, the staging buffer of one transposed
    (4-bit: dequantized) head chunk, bf16 [d][lce_head_t_ld(chunk)], and for a 4-bit head
    (`quantized`) the chunk's dequantized rows bf16 [chunk][d] after it."""
    chunk = min(chunk, -(-v // TILE) * TILE)
    rows = n if not row_block or row_block < 1 or row_block > n else row_block
    nchunks = -(-v // chunk)
    last_rows = n - (n - 1) // rows * rows
    last_tiles = -(-(v - (v - 1) // chunk * chunk) // TILE)
    parts = max(lce_dh_parts_bytes(r, d, kt) for r in (rows, last_rows) for kt in (chunk // TILE, last_tiles))
    total = rows * (chunk + G_PITCH_PAD) * 2 + (rows * d * 4 if nchunks > 1 else 0) + parts
    if staged:
        stage = d * lce_head_t_ld(chunk)
        if quantized:
            stage = -(-stage // 128) * 128 + chunk * d
        total = -(-total // 256) * 256 + stage * 2
    return total


def lce_head_t_ld(v: int) -> int:
    """Row pitch (elements) of a transposed head of v vocab rows: round_up(v, 256) + G_PITCH_PAD."""
    return -(-v // TILE) * TILE + G_PITCH_PAD


def lce_stage_chunk(n: int, d: int, v: int, budget: int, *, quantized: bool = False) -> int:
    """Vocab columns per chunk (multiple of 256) of the staged backward over all n rows: per
    column 2 n bytes of gradient tiles and 2 d of the staged head chunk (4 d for a 4-bit head, whose
    dequantized rows are staged too), plus the fp32 dH accumulator when the vocab takes more than
    one chunk, within the budget."""
    vpad = -(-v // TILE) * TILE
    per_col = 2 * (n + d) + (2 * d if quantized else 0)
    if per_col * (vpad + G_PITCH_PAD) <= budget:
        return vpad
    rest = max(budget - n * d * 4, 0)
    c = (rest // per_col - G_PITCH_PAD) // TILE * TILE
    return min(max(c, TILE), vpad)


@dataclass(frozen=True)
class LcePlan:
    fwd_splits: int
    fwd_workspace_bytes: int
    bwd_row_block: int
    bwd_row_blocks: int
    bwd_chunk: int
    bwd_chunks: int
    bwd_workspace_bytes: int


def lce_fwd_stages_whole_head(n: int, d: int, v: int, budget: int) -> bool:
    """The loss layer's staged 4-bit forward runs only when the whole dequantized head fits the
    budget (one launch over every vocab split)."""
    whole = -(-lce_fwd_workspace_bytes(n, v) // 256) * 256 + v * d * 2
    return d % 64 == 0 and lce_fwd_stage_workspace_bytes(n, d, v, budget) == whole


def lce_plan(*, n: int, v: int, d: int = 4096, budget: int | None = None, trainable: bool = False,
             staged: bool = False, quantized: bool = False, fwd_staged: bool = False) -> LcePlan:
    """Forward splits and backward geometry. A trainable head's dL/dW sums over every row, so its
    backward takes all rows in one block (the vocab is chunked instead when they do not fit); so
    does the staged backward (`staged`: a head without the cached transposed copy whose chunks are
    transposed into the workspace), whose chunks also carry the staged head chunk (and, for a 4-bit
    head, `quantized`, its dequantized rows). `fwd_staged`: the 4-bit forward that dequantizes runs
    of its vocab splits into its workspace (within the same budget)."""
    b = lce_bwd_budget_bytes() if budget is None else budget
    if staged:
        rows, chunk = n, lce_stage_chunk(n, d, v, b, quantized=quantized)
    else:
        rows = n if trainable else lce_bwd_row_block(n, d, v, b)
        chunk = -(-v // TILE) * TILE if rows < n else lce_bwd_chunk(n, d, v, b)
    fws = lce_fwd_stage_workspace_bytes(n, d, v, b) if fwd_staged else lce_fwd_workspace_bytes(n, v)
    return LcePlan(fwd_splits=lce_fwd_splits(n, v), fwd_workspace_bytes=fws,
                   bwd_row_block=rows, bwd_row_blocks=-(-n // rows), bwd_chunk=chunk, bwd_chunks=-(-v // chunk),
                   bwd_workspace_bytes=lce_bwd_workspace_bytes(n, d, v, chunk, rows, staged=staged,
                                                               quantized=staged and quantized))


def attn_heads_per_workgroup(hq: int, hkv: int) -> int:
    g = hq // hkv
    return 4 if g % 4 == 0 else (2 if g % 2 == 0 else 1)


def attn_dkv_splits(*, b: int, hq: int, hkv: int, s: int, dh: int = 128, causal: bool = True) -> int:
    """Workgroups per 128-key block of the dK/dV pass (every head_dim; `dh` only sizes the workspace): the size table of the launch
    plan (the MI355X counterpart of the reference's tile selection by sequence bucket,
    attention/kernel/dispatch.py:46-133), mirroring attn_dkv_nsplit in csrc/attn_kernels.hip.

    A key block's work is one item per (query head of its group, 64-query tile it sees): under the
    causal mask block kb sees the tiles from 128 kb on. One 8-wave workgroup runs per CU, so when
    the heaviest block exceeds ~1.15x a CU's share of all items (or blocks are fewer than CUs) the
    light CUs idle behind it; the block is then split over 2, 4 or 8 workgroups, the smallest count
    that brings the heaviest workgroup under the share, and their fp32 partials are summed."""
    if b < 1 or hkv < 1 or s < 1 or hq % hkv:
        return 1
    g = hq // hkv
    nkb = -(-s // 128)
    heaviest = g * -(-s // 64)
    total = b * hkv * sum(g * (-(-(s - 128 * kb) // 64) if causal else -(-s // 64)) for kb in range(nkb))
    for ns in (1, 2, 4):
        if heaviest * NUM_CU * 100 <= 115 * total * ns:
            return ns
    return 8


def attn_bwd_workspace_bytes(*, b: int, hq: int, hkv: int, s: int, dh: int = 128) -> int:
    """D (fp32 per query row, padded to 256 B), the fp32 dK/dV partials of the larger split of the
    two masks (when either splits), the two int32 work orders of a packed backward (one entry per
    dQ query block and one per 128-key dK/dV block) and its int32 segment end per position, each
    padded to 256 B (csrc/attn_kernels.hip attn_bwd_workspace)."""
    ns = max(attn_dkv_splits(b=b, hq=hq, hkv=hkv, s=s, dh=dh, causal=True),
             attn_dkv_splits(b=b, hq=hq, hkv=hkv, s=s, dh=dh, causal=False))

    def pad(x: int) -> int:
        return -(-x // 256) * 256

    rows = 32 * (4 // attn_heads_per_workgroup(hq, hkv))   # query positions per dQ workgroup
    parts = ns * 2 * b * hkv * s * dh * 4 if ns > 1 else 0
    return pad(b * hq * s * 4) + parts + pad(4 * b * -(-s // rows)) + pad(4 * b * -(-s // 128)) + pad(4 * b * s)


@dataclass(frozen=True)
class AttnPlan:
    heads_per_workgroup: int
    fwd_workgroups: int
    dkv_splits: int
    dkv_workgroups: int
    bwd_workspace_bytes: int


def attn_plan(*, b: int, hq: int, hkv: int, s: int, dh: int = 128, causal: bool = True) -> AttnPlan:
    hpw = attn_heads_per_workgroup(hq, hkv)
    p = 32 * (4 // hpw)
    ns = attn_dkv_splits(b=b, hq=hq, hkv=hkv, s=s, dh=dh, causal=causal)
    return AttnPlan(heads_per_workgroup=hpw, fwd_workgroups=-(-s // p) * b * (hq // hpw), dkv_splits=ns,
                    dkv_workgroups=-(-s // 128) * b * hkv * ns,
                    bwd_workspace_bytes=attn_bwd_workspace_bytes(b=b, hq=hq, hkv=hkv, s=s, dh=dh))
