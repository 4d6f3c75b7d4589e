"""Sequence packing producer: the wire format feeding packed attention and the packed loss
(torch counterpart of src/mlx_train_perf/data/packing.py:15-254).

The layout contract is the reference's, kept identical because the packed attention kernels and
the packed loss consume it:
- a sequence costs `min(len, pack_len) + 1` slots (its tokens plus one trailing pad slot it owns)
  against a row capacity of `pack_len + 1` (packing.py:15-48);
- packs are formed first-fit over a per-(seed, epoch) shuffle, scanning at most 8 open packs and
  closing a pack once at most one slot is left;
- inputs-axis arrays (`pack_len` wide): `seg_id` contiguous ascending from 0 per row, `seg_start`
  each position's segment start, a trailing tail segment covering unused capacity (gapless), and
  `loss_mask` supervising `[t0 + max(offset, 1) - 1, t0 + len - 1]` per segment
  (packing.py:102-156).
The shuffle uses Python's `random.Random(f"{seed}:{epoch}")`, so a given dataset packs the same
way as in the reference.
"""
from __future__ import annotations

import random
from collections.abc import Iterator, Sequence
from dataclasses import dataclass
from typing import Any

import torch

from mlx_train_perf.errors import PackingError

OPEN_POOL = 8  # open packs scanned by first-fit before the oldest is closed


def pack_indices(lengths: Sequence[int], pack_len: int, *, seed: int, epoch: int) -> list[list[int]]:
    """Group dataset indices into packs (deterministic per (seed, epoch))."""
    if pack_len < 1:
        raise PackingError(f"pack_len must be >= 1; got {pack_len}")
    if not lengths:
        raise PackingError("cannot pack an empty dataset")
    if min(lengths) < 1:
        raise PackingError("zero-length sequence in dataset")
    order = list(range(len(lengths)))
    random.Random(f"{seed}:{epoch}").shuffle(order)
    cap = pack_len + 1
    packs: list[list[int]] = []
    free: list[int] = []
    candidates: list[int] = []  # indices of packs still open, oldest first
    for idx in order:
        need = min(lengths[idx], pack_len) + 1
        target = next((p for p in candidates if free[p] >= need), None)
        if target is None:
            packs.append([idx])
            free.append(cap - need)
            candidates.append(len(packs) - 1)
            if len(candidates) > OPEN_POOL:
                del candidates[0]
            continue
        packs[target].append(idx)
        free[target] -= need
        if free[target] <= 1:  # nothing (not even a 1-token sequence + pad) fits any more
            candidates.remove(target)
    return packs


@dataclass(frozen=True, slots=True, kw_only=True)
class PackStats:
    real_tokens: int
    capacity_tokens: int
    utilization: float
    separator_fraction: float
    tail_pad_fraction: float


def pack_stats(packs: list[list[int]], lengths: Sequence[int], pack_len: int) -> PackStats:
    """Utilization over a `pack_len`-token row budget; the three fractions sum to 1 + 1/pack_len
    (each pack's `pack_len + 1` slots split into content, one pad per sequence and tail padding)."""
    if pack_len < 1:
        raise PackingError(f"pack_len must be >= 1; got {pack_len}")
    if not packs:
        raise PackingError("cannot compute stats over an empty pack list")
    real = sum(min(lengths[i], pack_len) for p in packs for i in p)
    seps = sum(len(p) for p in packs)
    tail = len(packs) * (pack_len + 1) - real - seps
    cap = len(packs) * pack_len
    return PackStats(real_tokens=real, capacity_tokens=cap, utilization=real / cap,
                     separator_fraction=seps / cap, tail_pad_fraction=tail / cap)


def build_row(entries: list[tuple[list[int], int]],
              pack_len: int) -> tuple[list[int], list[int], list[int], list[bool]]:
    """One packed row from `(tokens, offset)` entries: (row (pack_len+1), seg_id, seg_start,
    loss_mask (each pack_len))."""
    row = [0] * (pack_len + 1)
    seg_id = [0] * pack_len
    seg_start = [0] * pack_len
    loss_mask = [False] * pack_len
    pos = 0
    for sid, (tokens, offset) in enumerate(entries):
        n = len(tokens)
        row[pos:pos + n] = tokens
        last = min(pos + n, pack_len - 1)  # the segment's own pad slot, clipped to the inputs axis
        seg_id[pos:last + 1] = [sid] * (last + 1 - pos)
        seg_start[pos:last + 1] = [pos] * (last + 1 - pos)
        first_sup = pos + max(offset, 1) - 1
        for p in range(first_sup, pos + n):
            loss_mask[p] = True
        pos += n + 1
    if pos < pack_len:
        seg_id[pos:] = [len(entries)] * (pack_len - pos)
        seg_start[pos:] = [pos] * (pack_len - pos)
    return row, seg_id, seg_start, loss_mask


def packed_iterate_batches(dataset: Any, batch_size: int, max_seq_length: int, loop: bool = False,
                           seed: int | None = None, comm_group: Any = None, *,
                           max_position_embeddings: int | None = None,
                           device: str | torch.device | None = None,
                           ) -> Iterator[tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]]:
    """Yield `(batch int32 (B, L+1), seg_id int32 (B, L), seg_start int32 (B, L), loss_mask bool (B, L))`
    with `L = max_seq_length` (same shapes every step). Items are `(tokens, offset)` or bare tokens;
    overlong sequences are truncated with a one-time warning; a trailing partial batch is dropped.
    Refuses distributed packing (`comm_group.size() > 1`) and `max_seq_length > max_position_embeddings`."""
    if comm_group is not None and comm_group.size() > 1:
        raise PackingError(f"packed_iterate_batches does not support distributed packing "
                           f"(comm_group.size()={comm_group.size()}); pack on a single worker")
    if max_position_embeddings is not None and max_seq_length > max_position_embeddings:
        raise PackingError(f"max_seq_length={max_seq_length} exceeds max_position_embeddings={max_position_embeddings}")
    items: list[tuple[list[int], int]] = []
    for j in range(len(dataset)):
        entry = dataset[j]
        tokens, offset = entry if isinstance(entry, tuple) and len(entry) == 2 else (entry, 0)
        items.append((list(tokens), int(offset)))
    longest = max((len(t) for t, _ in items), default=0)
    if longest > max_seq_length:
        print(f"[WARNING] Some sequences are longer than {max_seq_length} tokens. The longest sentence {longest} "
              f"will be truncated to {max_seq_length}. Consider pre-splitting your data to save memory.")
    items = [(t[:max_seq_length], o) for t, o in items]
    lengths = [len(t) for t, _ in items]
    epoch = 0
    while True:
        packs = pack_indices(lengths, max_seq_length, seed=seed or 0, epoch=epoch)
        nb = len(packs) // batch_size
        if nb == 0:
            raise PackingError(f"packed dataset produced {len(packs)} pack(s) at pack_len={max_seq_length}, fewer than "
                               f"batch_size={batch_size}; reduce batch_size or add more data")
        for b in range(nb):
            rows = [build_row([items[i] for i in p], max_seq_length) for p in packs[b * batch_size:(b + 1) * batch_size]]
            yield (torch.tensor([r[0] for r in rows], dtype=torch.int32, device=device),
                   torch.tensor([r[1] for r in rows], dtype=torch.int32, device=device),
                   torch.tensor([r[2] for r in rows], dtype=torch.int32, device=device),
                   torch.tensor([r[3] for r in rows], dtype=torch.bool, device=device))
        epoch += 1
        if not loop:
            break
