"""Pins for oracle.sampling and oracle.slots.

* counter_uniform and sample_top_k_top_p_counter reproduce the golden vectors
  written from the reference's own functions (tests/golden/counter_sampling.npz,
  made by tests/golden/make_counter_sampling.py); the integer hash also matches
  an independent numpy uint32 evaluation;
* top_k = 1 is the argmax; top_p = 1 keeps the whole top-k;
* the fused top-20 sampler and the torch sampler agree on the token for rows
  whose threshold is not within rounding of a CDF boundary;
* the bookkeeping restatement agrees with the reference's torch fallback (a
  second formulation of the same step) over randomized multi-step scenarios;
* slot selection and cu_seqlens match their definitions.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sampling, slots

GOLD = np.load(Path(__file__).parent / "golden" / "counter_sampling.npz", allow_pickle=False)


def test_counter_uniform_golden():
    ids, steps = torch.from_numpy(GOLD["ids"]), torch.from_numpy(GOLD["steps"])
    for key in GOLD["uniform_keys"]:
        seed, stream = (int(x) for x in str(key).split("_"))
        u = sampling.counter_uniform(ids, steps, seed=seed, stream=stream)
        assert np.array_equal(u.numpy(), GOLD[f"uniform_{key}"])


def test_counter_word_matches_numpy_uint32():
    g = np.random.default_rng(0)
    ids = g.integers(0, 2**40, 500)
    steps = g.integers(0, 2**34, 500)
    w = sampling.counter_words_numpy(ids, steps, 20260923, 3)
    assert [sampling.counter_word(int(a), int(s), 20260923, 3) for a, s in zip(ids, steps)] == w.tolist()


def test_uniform_is_uniform():
    u = sampling.counter_uniform(torch.arange(20000), torch.zeros(20000, dtype=torch.long), seed=1)
    assert abs(u.double().mean().item() - 0.5) < 0.01 and abs(u.double().var().item() - 1 / 12) < 0.005
    assert (u > 0).all() and (u < 1).all()


def test_sampler_golden_tokens_and_distribution():
    logits = torch.from_numpy(GOLD["logits"])
    att, st = torch.from_numpy(GOLD["attempt_ids"]), torch.from_numpy(GOLD["row_steps"])
    for i, (t, k, p, seed) in enumerate(GOLD["sample_cases"].tolist()):
        tok = sampling.sample_top_k_top_p_counter(logits, att, st, seed=int(seed), temperature=t, top_k=int(k),
                                                  top_p=p)
        assert np.array_equal(tok.numpy(), GOLD[f"tokens_{i}"]), f"case {i}"
        if int(k) > 1:
            idx, probs = sampling.top_k_top_p_distribution(logits, temperature=t, top_k=int(k), top_p=p)
            assert np.array_equal(idx.numpy(), GOLD[f"dist_idx_{i}"])
            assert np.allclose(probs.numpy(), GOLD[f"dist_p_{i}"], atol=1e-7)


def test_sampler_full_vocabulary_golden_tokens():
    """The reference's full-vocabulary branches (inference_kernels.py:78-86)."""
    att, st = torch.from_numpy(GOLD["attempt_ids"]), torch.from_numpy(GOLD["row_steps"])
    for name, key in (("", "logits"), ("bf16_", "logits_bf16")):
        logits = torch.from_numpy(GOLD[key])
        for i, (t, k, p, seed) in enumerate(GOLD["full_cases"].tolist()):
            tok = sampling.sample_top_k_top_p_counter(logits, att, st, seed=int(seed), temperature=t,
                                                      top_k=int(k), top_p=p)
            assert np.array_equal(tok.numpy(), GOLD[f"full_{name}tokens_{i}"]), f"{name}case {i}"


def test_sampler_special_cases():
    logits = torch.from_numpy(GOLD["logits"])
    att, st = torch.from_numpy(GOLD["attempt_ids"]), torch.from_numpy(GOLD["row_steps"])
    tok = sampling.sample_top_k_top_p_counter(logits, att, st, seed=1, temperature=0.7, top_k=1, top_p=0.9)
    assert torch.equal(tok[:, 0], logits.argmax(-1))
    idx, p = sampling.top_k_top_p_distribution(logits, temperature=1.0, top_k=8, top_p=1.0)
    assert (p > 0).all()  # top_p = 1 keeps every top-k candidate


def test_fused_and_torch_samplers_agree_away_from_ties():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(64, 300, generator=g) * 2
    att = torch.arange(64)
    steps = torch.randint(0, 1000, (64,), generator=g)
    vals, idx = torch.topk(logits, 20)
    fused = sampling.top20_counter_sample(vals / 0.6, idx, att, steps, seed=11, top_p=0.95)
    tor = sampling.sample_top_k_top_p_counter(logits, att, steps, seed=11, temperature=0.6, top_k=20, top_p=0.95)
    assert (fused == tor).float().mean().item() > 0.95


def _top20_exact_ranks(values, attempt_ids, steps, seed, top_p, prefix_rule="before"):
    """The fused top-20 rule in float64 (softmax, keep p while the mass before it
    is below top_p, threshold u * retained, rank = #(cumulative < threshold)),
    with the margin of each row to its nearest decision boundary."""
    v = values.double()
    p = torch.softmax(v, dim=-1)
    cum_all = p.cumsum(-1)
    before = cum_all - p if prefix_rule == "before" else cum_all
    keep = before < top_p
    trunc = torch.where(keep, p, torch.zeros_like(p))
    retained = trunc.sum(-1, keepdim=True)
    cum = trunc.cumsum(-1)
    u = torch.tensor([(sampling.counter_word(int(a), int(t), seed) + 0.5) / 4294967296.0
                      for a, t in zip(attempt_ids.tolist(), steps.tolist())], dtype=torch.float64)[:, None]
    thr = u * retained
    rank = (cum < thr).sum(-1).clamp_max(values.shape[-1] - 1)
    margin = torch.minimum((before - top_p).abs().min(-1).values, ((cum - thr).abs() / retained).min(-1).values)
    return rank, margin


def test_top20_sampler_matches_exact_rule_away_from_boundaries():
    """Pins the fused top-20 restatement (inference_kernels.py:1119-1145) to
    the same rule evaluated in float64: on every row whose threshold and top-p
    cut sit more than 1e-5 from a cumulative boundary, the float32 restatement
    picks the same rank.  Varied temperatures, top_p in (0, 1] and heavy/flat
    rows; a planted mistake (keep p while cumsum(p), not the mass before p, is
    below top_p) must fail the same check."""
    g = torch.Generator().manual_seed(19)
    rows = 512
    logits = torch.randn(rows, 1000, generator=g) * torch.linspace(0.2, 6.0, rows)[:, None]
    att = torch.randint(0, 1 << 31, (rows,), generator=g)
    steps = torch.randint(0, 1 << 20, (rows,), generator=g)
    vals, idx = torch.topk(logits, 20)
    checked = 0
    for top_p, temp in ((0.95, 0.6), (0.5, 1.0), (1.0, 0.8), (0.05, 1.3)):
        scaled = vals / temp
        got = sampling.top20_counter_sample(scaled, idx, att, steps, seed=7, top_p=top_p)[:, 0]
        rank, margin = _top20_exact_ranks(scaled, att, steps, 7, top_p)
        want = idx.gather(1, rank[:, None])[:, 0]
        ok = margin > 1e-5
        checked += int(ok.sum())
        assert torch.equal(got[ok], want[ok]), top_p
        if 0.1 < top_p < 1.0:  # (at top_p 0.05 both rules keep only the top candidate)
            bad_rank, _ = _top20_exact_ranks(scaled, att, steps, 7, top_p, prefix_rule="cumsum")
            assert not torch.equal(got[ok], idx.gather(1, bad_rank[:, None])[:, 0][ok]), top_p
    assert checked > 0.9 * 4 * rows


def _bookkeeping_scenario(seed, slots_n=12, attempts=20, width=9, vocab=50):
    g = torch.Generator().manual_seed(seed)
    st = dict(
        sampled=torch.randint(0, vocab, (slots_n, 1), generator=g),
        storage=torch.full((attempts + slots_n, width + 1), 7, dtype=torch.int32),
        dense_seen=torch.rand(slots_n, vocab, generator=g) < 0.1,
        generated_lengths=torch.randint(0, 3, (attempts + slots_n,), generator=g),
        finished_by_eos=torch.zeros(attempts + slots_n, dtype=torch.bool),
        finished=torch.rand(slots_n, generator=g) < 0.2,
        slot_rows=torch.where(torch.rand(slots_n, generator=g) < 0.85, torch.randperm(attempts, generator=g)[:slots_n],
                              torch.tensor(-1)),
        sink_rows=attempts + torch.arange(slots_n),
        slot_caps=torch.randint(2, width, (slots_n,), generator=g),
        row_steps=torch.randint(1, 3, (slots_n,), generator=g),
        row_positions=torch.randint(5, 50, (slots_n,), generator=g),
        decode_ids=torch.zeros(slots_n, 1, dtype=torch.long),
        useful=torch.zeros((), dtype=torch.long),
    )
    return st, g


@pytest.mark.parametrize("seed", range(5))
def test_bookkeeping_matches_reference_fallback(seed):
    a, g = _bookkeeping_scenario(seed)
    b = {k: v.clone() for k, v in a.items()}
    kw = dict(maximum_new_tokens=9, pad_token_id=7, eos_token_ids=(3, 4))
    for step in range(8):
        tok = torch.randint(0, 50, (12, 1), generator=g)
        a["sampled"], b["sampled"] = tok.clone(), tok.clone()
        slots.decode_state_update(*a.values(), **kw)
        slots.decode_state_update_torch(*b.values(), **kw)
        for k in a:
            assert torch.equal(a[k], b[k]), f"{k} differs at step {step}"


def test_selection_and_cu_seqlens():
    fin = torch.tensor([True, False, False, True, False])
    rows = torch.tensor([3, -1, 5, 2, 0])
    assert slots.refill_targets(fin) == [0, 3]
    assert slots.compaction_keep(fin, rows) == [2, 4]
    assert slots.cu_seqlens([5, 0, 2]) == [0, 5, 5, 7]
    assert slots.should_compact(3, 8, queue_exhausted=True, live_fraction=0.5)
    assert not slots.should_compact(5, 8, queue_exhausted=True, live_fraction=0.5)
    assert not slots.should_compact(3, 8, queue_exhausted=False, live_fraction=0.5)
