"""Packing producer (CPU): the reference's hand-worked layout examples
(tests/test_packing.py:106-131 of the reference), stats KATs, invariants and iterator contract."""
from __future__ import annotations

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from mlx_train_perf.data.packing import build_row, pack_indices, pack_stats, packed_iterate_batches
from mlx_train_perf.errors import PackingError


@settings(max_examples=60, deadline=None)
@given(st.lists(st.integers(1, 300), min_size=1, max_size=200), st.integers(0, 3), st.integers(0, 2))
def test_every_sequence_placed_once_and_capacity(lengths, seed, epoch):
    packs = pack_indices(lengths, 1024, seed=seed, epoch=epoch)
    assert sorted(i for p in packs for i in p) == list(range(len(lengths)))
    for p in packs:
        assert sum(min(lengths[i], 1024) + 1 for i in p) <= 1025


def test_deterministic_per_seed_epoch_and_varies_across_epochs():
    lengths = list(range(1, 120))
    a = pack_indices(lengths, 256, seed=7, epoch=0)
    assert a == pack_indices(lengths, 256, seed=7, epoch=0)
    assert a != pack_indices(lengths, 256, seed=7, epoch=1)


def test_refusals():
    for args in (([], 256), ([0, 5], 256), ([5], 0)):
        with pytest.raises(PackingError):
            pack_indices(args[0], args[1], seed=0, epoch=0)


def test_stats_hand_computed():
    s = pack_stats([[0], [1]], [15, 3], 10)
    assert (s.real_tokens, s.capacity_tokens) == (13, 20)
    assert s.utilization == pytest.approx(13 / 20) and s.separator_fraction == pytest.approx(2 / 20)
    assert s.tail_pad_fraction == pytest.approx(7 / 20)
    s = pack_stats([[0, 1], [2]], [5, 4, 9], 12)
    assert (s.real_tokens, s.capacity_tokens) == (18, 24)
    assert s.separator_fraction == pytest.approx(3 / 24) and s.tail_pad_fraction == pytest.approx(5 / 24)


def test_build_row_worked_example():
    row, seg_id, seg_start, loss_mask = build_row([([10, 11, 12, 13, 14], 2), ([20, 21, 22, 23], 1)], pack_len=12)
    assert row == [10, 11, 12, 13, 14, 0, 20, 21, 22, 23, 0, 0, 0]
    assert seg_id == [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2]
    assert seg_start == [0, 0, 0, 0, 0, 0, 6, 6, 6, 6, 6, 11]
    assert loss_mask == [False, True, True, True, True, False, True, True, True, True, False, False]


def test_build_row_offset_zero_supervises_from_position_zero():
    _, _, _, m = build_row([([5, 6, 7], 0)], pack_len=8)
    assert m[:3] == [True, True, True]


@settings(max_examples=80, deadline=None)
@given(entries=st.lists(st.tuples(st.lists(st.integers(1, 1000), min_size=1, max_size=6), st.integers(0, 5)),
                        min_size=0, max_size=5), slack=st.integers(0, 5))
def test_gapless_coverage_and_monotone(entries, slack):
    pack_len = max(sum(len(t) + 1 for t, _ in entries) - 1 + slack, 1)
    row, seg_id, seg_start, loss_mask = build_row(entries, pack_len)
    assert len(row) == pack_len + 1 and len(seg_id) == len(seg_start) == len(loss_mask) == pack_len
    assert seg_id == sorted(seg_id)
    for i in range(pack_len):
        assert 0 <= seg_start[i] <= i and seg_id[seg_start[i]] == seg_id[i]
        if i and seg_id[i] != seg_id[i - 1]:
            assert seg_start[i] == i


def test_iterator_shapes_dtypes_and_refusals(capsys):
    it = packed_iterate_batches(dataset=[([1, 2, 3, 4], 1)] * 8, batch_size=2, max_seq_length=16, seed=3)
    batch, sid, sst, lm = next(it)
    assert batch.shape == (2, 17) and sid.shape == sst.shape == lm.shape == (2, 16)
    assert batch.dtype == sid.dtype == sst.dtype == torch.int32 and lm.dtype == torch.bool

    class Group:
        def __init__(self, n):
            self.n = n

        def size(self):
            return self.n

    with pytest.raises(PackingError):
        next(packed_iterate_batches(dataset=[([1, 2], 0)] * 4, batch_size=2, max_seq_length=8, comm_group=Group(2)))
    next(packed_iterate_batches(dataset=[([1, 2, 3], 0)] * 4, batch_size=2, max_seq_length=8, comm_group=Group(1)))
    with pytest.raises(PackingError):
        next(packed_iterate_batches(dataset=[[1, 2]] * 4, batch_size=2, max_seq_length=64, max_position_embeddings=32))
    with pytest.raises(PackingError):
        next(packed_iterate_batches(dataset=[[1, 2]], batch_size=2, max_seq_length=8))
    out = next(packed_iterate_batches(dataset=[list(range(1, 30))] * 4, batch_size=1, max_seq_length=10))
    assert "truncated to 10" in capsys.readouterr().out and out[0].shape == (1, 11)


def test_bare_items_and_epoch_reshuffle():
    ds = [[i + 1] * (1 + i % 5) for i in range(40)]
    it = packed_iterate_batches(dataset=ds, batch_size=1, max_seq_length=8, loop=True, seed=1)
    first_epoch = [next(it)[0] for _ in range(len(pack_indices([len(x) for x in ds], 8, seed=1, epoch=0)))]
    second = next(it)[0]
    assert any(not torch.equal(second, f) for f in first_epoch[:1])
