"""Host-side scheduling logic of the runtime (CPU).

* ``_initial_attempt_order`` (runtime/model/inference_kernels.py:1321-1329):
  hand-worked cases, with and without prefill groups;
* ``_should_compact_dynamic_decode_tail`` (1348-1349): the boundary cases;
* ``synthetic_requests``: the backlog that fills the batch arrives at step 0.
"""
import torch

from yanchor_amd import inference_kernels as ik
from yanchor_amd import runtime as rt


def test_initial_attempt_order_without_groups():
    # caps (difficulty) 5, 9, 9, 1 for attempts 30, 20, 10, 40:
    # largest cap first; the two caps of 9 ordered by attempt id (10 before 20)
    assert ik._initial_attempt_order([5, 9, 9, 1], [30, 20, 10, 40]) == [2, 1, 0, 3]
    assert ik._initial_attempt_order(torch.tensor([2.0, 2.0, 2.0]), [7, 3, 5]) == [1, 2, 0]
    assert ik._initial_attempt_order([], []) == []


def test_initial_attempt_order_with_groups():
    # rows:        0   1   2   3   4
    # difficulty:  1   8   3   8   2
    # attempt id:  4   3   2   1   0
    # group:      10  10  11  12  11
    # group 10: max 8, min id 3; group 12: max 8, min id 1; group 11: max 3, min id 0
    # -> 12, 10, 11; inside 10: row 1 (8) then row 0 (1); inside 11: row 2 (3), row 4 (2)
    order = ik._initial_attempt_order([1, 8, 3, 8, 2], [4, 3, 2, 1, 0], [10, 10, 11, 12, 11])
    assert order == [3, 1, 0, 2, 4]
    from oracle import slots
    assert slots.initial_attempt_order([1, 8, 3, 8, 2], [4, 3, 2, 1, 0], [10, 10, 11, 12, 11]) == order
    assert slots.initial_attempt_order([5, 9, 9, 1], [30, 20, 10, 40]) == [2, 1, 0, 3]


def test_group_aligned_prefix_and_expansion():
    """_group_aligned_prefix_length (inference_kernels.py:1331-1346) and
    build_prefill_expansion (90-121): hand-worked cases, product and oracle."""
    from oracle import slots
    order, groups = [3, 1, 0, 2, 4], [10, 10, 11, 12, 11]     # groups along the order: 12 | 10 10 | 11 11
    for f in (ik._group_aligned_prefix_length, slots.group_aligned_prefix):
        assert [f(order, groups, k) for k in (1, 2, 3, 4, 5, 9)] == [1, 1, 3, 3, 5, 5]
        assert f([], groups, 3) == 0 and f(order, groups, 0) == 0
    import pytest
    with pytest.raises(ValueError):
        ik._group_aligned_prefix_length([1, 0, 3], groups, 1)    # group 10 holds two rows
    with pytest.raises(ValueError):
        slots.group_aligned_prefix([1, 0, 3], groups, 1)
    assert slots.prefill_expansion([7, 3, 7, 9, 3]) == ([0, 1, 3], [0, 1, 0, 2, 1])


def test_tail_compaction_trigger():
    f = ik._should_compact_dynamic_decode_tail
    assert f(64, 128, queue_exhausted=True, live_fraction=0.5)
    assert not f(65, 128, queue_exhausted=True, live_fraction=0.5)
    assert not f(64, 128, queue_exhausted=False, live_fraction=0.5)
    assert not f(0, 128, queue_exhausted=True, live_fraction=0.5)
    assert not f(1, 1, queue_exhausted=True, live_fraction=0.5)
    assert f(1, 3, queue_exhausted=True, live_fraction=0.1)     # max(1, int(0.3)) = 1


def test_synthetic_requests_backlog():
    reqs = rt.synthetic_requests(10, rate=4.0, prompt_len=8, vocab=100, initial=128)
    at0 = [r for r in reqs if r.arrival_step == 0]
    assert len(at0) >= 128
    assert [r.attempt_id for r in reqs] == list(range(len(reqs)))
    assert all(r.prompt.shape == (8,) and 1 <= r.cap <= 8192 for r in reqs)
    # the same seed without the backlog gives the same Poisson arrivals after step 0
    plain = rt.synthetic_requests(10, rate=4.0, prompt_len=8, vocab=100)
    assert sum(r.arrival_step > 0 for r in plain) == sum(r.arrival_step > 0 for r in reqs)


def test_repetition_periods():
    """The mechanical-repetition stop (runtime/scoring/protocols.py:89-109):
    the smallest period in [128, 256] whose 8 copies end the sequence."""
    import numpy as np
    rng = np.random.default_rng(0)
    unit = rng.integers(0, 1000, 130)
    w = 256 * 8
    rows, lengths = [], []

    def right_aligned(seq):
        row = np.zeros(w, dtype=np.int64)
        row[w - len(seq):] = seq
        return row

    rep = np.concatenate([rng.integers(0, 1000, 50), np.tile(unit, 8)])         # 8 copies of a 130-block
    rows.append(right_aligned(rep)), lengths.append(len(rep))
    rows.append(right_aligned(np.tile(unit, 7))), lengths.append(130 * 7)       # only 7 copies
    short = rng.integers(0, 1000, 100)
    rows.append(right_aligned(np.tile(short, 16))), lengths.append(1600)       # period 100 < 128: its double 200 counts
    rows.append(right_aligned(rng.integers(0, 1000, w))), lengths.append(w)    # no repetition
    rows.append(right_aligned(np.tile(np.arange(128), 8))), lengths.append(1024)
    got = rt.repetition_periods(np.stack(rows), np.array(lengths))
    assert got.tolist() == [130, 0, 200, 0, 128]
    assert rt.repetition_periods(np.zeros((1, 100), dtype=np.int64), np.array([100])).tolist() == [0]


def test_text_ids_round_trip():
    from yanchor_amd import inference
    ids = inference.encode_text("héllo, world", 151936)
    assert all(0 <= i < 256 for i in ids)
    assert inference.decode_ids(ids) == "héllo, world"
    assert inference.decode_ids([104, 105, 5000]) == "hi�"
