"""Host model of the LCE GEMM core's LDS stage hand-off (csrc/lce_kernels.hip `gemm_dma` and the
per-tile loops of `lce_fwd_kernel` / `lce_bwd_g_persist_kernel` that call it), CPU lane.

Two 64 KiB stage buffers alternate: stage kt of a tile lives in buffer kt & 1. Between barriers
("epochs") the waves read one stage and the copier waves issue the copies of a later one; every copy
issued in an epoch has landed by the barrier that ends it (each copier waits for its copies before
the barrier), except the prologue's stage-1 copies, which the first wait leaves in flight until the
barrier after stage 0 (`wait_vmcnt<8>`). A workgroup that walks several tiles prefetches the next
tile's stages 0 and 1 after the last barrier (`next`), and, when both tiles are whole and nk is
even, issues the next tile's stage 0 early, in the copy slot of stage nk (past the end) right after
barrier nk - 2 (`early0`, `next_shift`).

The model replays that schedule for three consecutive tiles and checks, for every nk, with and
without the early stage 0:
  - every read finds the stage it expects in its buffer, written by copies that landed by a barrier
    before the read's epoch (no read-before-write);
  - no copy is issued into a buffer in an epoch in which some wave reads that buffer, or before a
    later read of what the buffer held (no write-after-read race).
Planted mistakes (the early stage 0 with nk odd; the stage copies issued before the barrier instead
of after it; the next tile's prefetch issued before the last barrier) must fail the same checks.
"""
from __future__ import annotations

import pytest


def _schedule(nk: int, tiles: int, *, early0_allowed: bool = True, copy_before_barrier: bool = False,
              next_before_last_barrier: bool = False, force_early0: bool = False):
    """Events (epoch, kind, buffer, label, landed_epoch) of `tiles` consecutive tiles.
    kind 'r' = a wave reads `label` from `buffer`; 'c' = a copy of `label` into `buffer`, issued in
    `epoch`, landed by the start of `landed_epoch`."""
    ev = []
    e = 0  # current epoch
    pre = False
    for t in range(tiles):
        has_next = t + 1 < tiles
        early0 = force_early0 or (early0_allowed and has_next and nk % 2 == 0)
        if not pre:
            ev.append((e, "c", 0, (t, 0), e + 1))
            if nk > 1:
                ev.append((e, "c", 1, (t, 1), e + 2))   # wait_vmcnt<8>: lands by barrier B_0
        e += 1                                          # prologue barrier
        ev.append((e, "r", 0, (t, 0), None))            # stage 0, k-step 0
        for kt in range(nk - 1):
            cur, nxt = kt & 1, (kt + 1) & 1
            ev.append((e, "r", cur, (t, kt), None))     # k-steps 1-3 of stage kt
            if copy_before_barrier and kt + 2 < nk:
                ev.append((e, "c", cur, (t, kt + 2), e + 1))
            e += 1                                      # barrier B_kt (after the waits)
            if not copy_before_barrier and kt + 2 < nk:
                ev.append((e, "c", cur, (t, kt + 2), e + 1))
            elif kt + 2 == nk and early0:
                ev.append((e, "c", cur, (t + 1, 0), e + 1))  # next tile's stage 0 in the dead slot
            ev.append((e, "r", nxt, (t, kt + 1), None))  # k-step 0 of stage kt + 1
        last = (nk - 1) & 1
        ev.append((e, "r", last, (t, nk - 1), None))    # k-steps 1-3 of the last stage
        if has_next and next_before_last_barrier:
            if not early0:
                ev.append((e, "c", 0, (t + 1, 0), e + 1))
            if nk > 1:
                ev.append((e, "c", 1, (t + 1, 1), e + 1))
        e += 1                                          # last barrier
        if has_next and not next_before_last_barrier:
            if not early0:
                ev.append((e, "c", 0, (t + 1, 0), e + 1))
            if nk > 1:
                ev.append((e, "c", 1, (t + 1, 1), e + 1))
        # epilogue (no LDS), then the next call waits for its prefetched copies and barriers
        pre = has_next
    return ev


def _violations(ev) -> list[str]:
    bad = []
    copies = [x for x in ev if x[1] == "c"]
    reads = [x for x in ev if x[1] == "r"]
    for (e, _, b, lab, _) in reads:
        # the copy that provides what this read sees: the latest copy into b issued before epoch e
        prior = [c for c in copies if c[2] == b and c[0] < e]
        if not prior:
            bad.append(f"epoch {e}: read of {lab} from buffer {b} before any copy into it")
            continue
        src = max(prior, key=lambda c: c[0])
        if src[3] != lab:
            bad.append(f"epoch {e}: read of {lab} from buffer {b} finds {src[3]}")
        elif src[4] > e:
            bad.append(f"epoch {e}: read of {lab} from buffer {b} before its copy lands (epoch {src[4]})")
        # and no copy into b is issued in the read's own epoch (the waves are not ordered inside it)
        for c in copies:
            if c[2] == b and c[0] == e and c[3] != lab:
                bad.append(f"epoch {e}: copy of {c[3]} into buffer {b} races the read of {lab}")
    return bad


@pytest.mark.parametrize("nk", [1, 2, 3, 4, 5, 6, 7, 8, 64])
@pytest.mark.parametrize("early0", [False, True])
def test_stage_hand_off_has_no_races(nk, early0):
    ev = _schedule(nk, tiles=3, early0_allowed=early0)
    assert not _violations(ev), _violations(ev)
    # every stage of every tile is read
    read = {x[3] for x in ev if x[1] == "r"}
    assert read == {(t, s) for t in range(3) for s in range(nk)}


@pytest.mark.parametrize("nk", [3, 5, 7])
def test_early_stage0_with_odd_nk_is_caught(nk):
    """With nk odd the dead slot is buffer 1: the next tile's stage 0 would land where it is not read
    (and over its stage 1): the reason the kernels take the early stage 0 only when nk is even."""
    assert _violations(_schedule(nk, tiles=3, force_early0=True))


@pytest.mark.parametrize("nk", [3, 4, 6])
def test_copy_before_the_barrier_is_caught(nk):
    assert _violations(_schedule(nk, tiles=2, copy_before_barrier=True))


@pytest.mark.parametrize("nk", [2, 3, 4])
def test_prefetch_before_the_last_barrier_is_caught(nk):
    assert _violations(_schedule(nk, tiles=2, early0_allowed=False, next_before_last_barrier=True))
