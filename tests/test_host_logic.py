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
