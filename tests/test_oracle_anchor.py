"""Pins for oracle.anchor.

* the tensor select_topk / merge_topk (the reference's two stable sorts) agree
  with the brute-force sorted() selection on random candidates with forced
  score ties, -0.0 vs +0.0, -inf scores and dead slots;
* a selection that drops the position tie-break (a plausible mistake) is
  caught on a crafted tie;
* the committed read equals an independent formulation -- SDPA over
  [K; 0], [V; 0] with mask [live; True], the reference's own _gqa_tile
  construction (modeling_yanchor.py:22-32) -- and closed forms for zero and one
  live slot;
* exclusive_prefix_topk's definition form satisfies its recursion
  prefix[j+1] = merge(prefix[j], block j).
"""
import math

import pytest
import torch

from oracle import anchor
from oracle.anchor import MemoryState
from yanchor_amd import workloads


def _cands(n, seed, ties=True):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(n, generator=g)
    if ties:
        s = (s * 2).round() / 2  # many exact ties
    s[torch.rand(n, generator=g) < 0.1] = -math.inf
    z = torch.rand(n, generator=g) < 0.1
    s[z] = torch.where(torch.rand(int(z.sum()), generator=g) < 0.5, torch.tensor(0.0), torch.tensor(-0.0))
    p = torch.randperm(4 * n, generator=g)[:n].long()
    r = torch.arange(n)
    r[torch.rand(n, generator=g) < 0.2] = -1
    return s, p, r


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("cap", [5, 32, 64])
def test_tensor_select_matches_bruteforce(seed, cap):
    s, p, r = _cands(96, seed)
    ts, tp, tr = anchor.select_topk(s[None], p[None], r[None], cap)
    bs, bp, br = anchor.select_topk_bruteforce(s, p, r, cap)
    assert tr[0].tolist() == br and tp[0].tolist() == bp
    assert torch.equal(ts[0], torch.tensor(bs, dtype=ts.dtype))


def test_merge_pads_when_short():
    s, p, r = _cands(3, 1)
    out = anchor.merge_topk((s[None, :1], p[None, :1], r[None, :1]), (s[None, 1:], p[None, 1:], r[None, 1:]), 6)
    assert out[0].shape == (1, 6) and out[2][0, 3:].tolist() == [-1, -1, -1]
    assert out[1][0, 3:].tolist() == [-1, -1, -1]


def test_position_tiebreak_matters():
    """Equal scores: the earlier position wins, not the earlier index."""
    s = torch.tensor([1.0, 1.0, 1.0])
    p = torch.tensor([30, 10, 20])
    r = torch.tensor([0, 1, 2])
    _, _, ref = anchor.select_topk_bruteforce(s, p, r, 2)
    assert ref == [1, 2]
    wrong = sorted(range(3), key=lambda i: (-s[i].item(), i))[:2]  # index tie-break only
    assert wrong != ref


def test_negative_zero_ties_with_zero():
    s = torch.tensor([-0.0, 0.0])
    p = torch.tensor([5, 3])
    r = torch.tensor([0, 1])
    _, _, ref = anchor.select_topk_bruteforce(s, p, r, 1)
    assert ref == [1]  # tie on score (-0 == +0), position 3 first


def _sdpa_read(query, st):
    """The reference's _gqa_tile construction with torch SDPA (float64)."""
    b, _, h, d = query.shape
    g, cap = st.keys.shape[1:3]
    key = torch.nn.functional.pad(st.keys.double(), (0, 0, 0, 1))      # zero sink key
    val = torch.nn.functional.pad(st.values.double(), (0, 0, 0, 1))    # zero sink value
    mask = torch.nn.functional.pad(st.positions >= 0, (0, 1), value=True)
    q = query.double().reshape(b, g, h // g, d)
    out = torch.nn.functional.scaled_dot_product_attention(q, key, val, attn_mask=mask[:, :, None, :])
    return out.reshape(b, 1, h, d)


@pytest.mark.parametrize("r", [1, 2])
def test_read_matches_sdpa_with_sink(r):
    st = workloads.anchor_state(3, 2, 64, 8, 16, dtype=torch.float64, seed=4)
    q = workloads.anchor_query(3, 2 * r, 16, dtype=torch.float64, seed=5)
    got = anchor.committed_read(q, st)
    assert torch.allclose(got, _sdpa_read(q, st), atol=1e-12)


def test_read_closed_forms():
    st = workloads.anchor_state(1, 1, 64, 8, 8, dtype=torch.float64, seed=6)
    q = workloads.anchor_query(1, 1, 8, dtype=torch.float64, seed=7)
    st.positions.fill_(-1)
    assert torch.count_nonzero(anchor.committed_read(q, st)) == 0   # only the sink
    st.positions[0, 0, 17] = 3
    logit = (q[0, 0, 0] @ st.keys[0, 0, 17]).item() / math.sqrt(8)
    p = math.exp(logit) / (math.exp(logit) + 1.0)
    assert torch.allclose(anchor.committed_read(q, st)[0, 0, 0], p * st.values[0, 0, 17], atol=1e-12)


def test_read_skips_negative_index_rows():
    st = workloads.anchor_state(2, 1, 64, 8, 8, dtype=torch.float64, seed=8)
    q = workloads.anchor_query(2, 1, 8, dtype=torch.float64, seed=9)
    out = anchor.committed_read(q, st, torch.tensor([1, -1]))
    assert torch.count_nonzero(out[1]) == 0
    assert torch.allclose(out[0], anchor.committed_read(q[:1], MemoryState(
        *(getattr(st, f)[1:2] for f in MemoryState.__dataclass_fields__)))[0])


def test_commit_keeps_topk_of_union():
    """After a full chunk the committed slots are exactly the Top-K of
    committed + pending by (score desc, position, index), with K/V rows moved
    along; merge_topk (the reference's tensor path) selects the same."""
    cap, c, d = 16, 4, 8
    st = workloads.anchor_state(1, 2, cap, c, d, dtype=torch.float32, seed=10, fill_pending=c - 1, total0=100)
    before = MemoryState(*(getattr(st, f).clone() for f in MemoryState.__dataclass_fields__))
    g = torch.Generator().manual_seed(11)
    key, val = torch.randn(1, 1, 2, d, generator=g), torch.randn(1, 1, 2, d, generator=g)
    sc = torch.randn(1, 1, 2, generator=g)
    anchor.commit_decode(key, val, sc, torch.tensor([True]), c, st)
    assert st.count.item() == 0 and st.total.item() == 101
    for grp in range(2):
        cs = torch.cat((before.scores[0, grp], before.pending_scores[0, grp, :c - 1], sc[0, 0, grp:grp + 1]))
        cp = torch.cat((before.positions[0, grp].long(), 100 - (c - 1) + torch.arange(c)))
        cr = torch.cat((torch.arange(cap).masked_fill(before.positions[0, grp] < 0, -1), cap + torch.arange(c)))
        ts, tp, tr = anchor.select_topk(cs[None], cp[None], cr[None], cap)
        assert st.positions[0, grp].tolist() == tp[0].tolist()
        assert torch.equal(st.scores[0, grp], ts[0])
        src = torch.cat((before.keys[0, grp], before.pending_keys[0, grp, :c - 1], key[0, 0, grp:grp + 1]))
        assert torch.equal(st.keys[0, grp], src[tr[0].clamp_min(0)])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_batched_read_and_commit_equal_per_row(dtype):
    """The batched decode read / commit (the host CPU baseline's form) equal
    the per-row restatements over 40 steps: rows at staggered points of their
    chunk (so a few commit at every step), some slots dead, tied scores, one
    row inactive at times.  The state is bit-exact; the reads agree to the
    float32 rounding of the batched products."""
    b, g, cap, c, d, h = 6, 2, 16, 8, 16, 4
    st = workloads.anchor_state(b, g, cap, c, d, dtype=dtype, seed=21, p_live=0.6)
    st.count.copy_(torch.tensor([0, 3, 7, 5, 6, 1]))
    st.total.copy_(4 * cap + st.count)
    one = MemoryState(*(getattr(st, f).clone() for f in MemoryState.__dataclass_fields__))
    two = MemoryState(*(getattr(st, f).clone() for f in MemoryState.__dataclass_fields__))
    gen = torch.Generator().manual_seed(22)
    commits = 0
    for step in range(40):
        q = torch.randn(b, 1, h, d, generator=gen).to(dtype)
        key, val = torch.randn(b, 1, g, d, generator=gen).to(dtype), torch.randn(b, 1, g, d, generator=gen).to(dtype)
        sc = torch.randint(-2, 3, (b, 1, g), generator=gen).float()   # integer scores: ties
        active = torch.ones(b, dtype=torch.bool)
        active[step % b] = step % 3 != 0
        commits += int(((one.count + active.long()) == c).sum())
        r1 = anchor.committed_read(q, one, dtype=torch.float32)
        r2 = anchor.committed_read_batched(q, two)
        assert torch.allclose(r1.float(), r2.float(), rtol=1e-5, atol=1e-6 if dtype == torch.float32 else 1e-2)
        anchor.commit_decode(key, val, sc, active, c, one)
        anchor.commit_decode_batched(key, val, sc, active, c, two)
        for f in MemoryState.__dataclass_fields__:
            assert torch.equal(getattr(one, f), getattr(two, f)), (step, f)
    assert commits >= 25


def test_prefix_topk_recursion():
    b, nb, g, c, cap = 1, 5, 2, 4, 6
    gen = torch.Generator().manual_seed(12)
    s = (torch.randn(b, nb, g, c, generator=gen) * 2).round()
    p = torch.arange(nb * c).reshape(1, nb, 1, c).expand(b, nb, g, c).clone()
    r = p.clone()
    ps, pp, pr = anchor.exclusive_prefix_topk(s, p, r, cap)
    assert (pr[:, 0] == -1).all()
    for j in range(nb):
        nxt = anchor.merge_topk((ps[:, j], pp[:, j], pr[:, j]), (s[:, j], p[:, j], r[:, j]), cap)
        assert torch.equal(nxt[2], pr[:, j + 1]) and torch.equal(nxt[0], ps[:, j + 1])


def _prefill_inputs(b, nb, c, h, g, d, s, cap, kb, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, nb, c, h, d, generator=gen, dtype=torch.float64)
    k = torch.randn(kb, s, g, d, generator=gen, dtype=torch.float64)
    v = torch.randn(kb, s, g, d, generator=gen, dtype=torch.float64)
    refs = torch.randint(0, s, (b, nb, g, cap), generator=gen)
    refs[torch.rand(b, nb, g, cap, generator=gen) < 0.3] = -1
    return q, k, v, refs


@pytest.mark.parametrize("kb", [1, 2])
def test_indexed_read_matches_sdpa_over_gathered_rows(kb):
    """The _gqa_tile construction: gather the referenced rows, append a zero
    key / value row that is always visible, mask dead references, SDPA."""
    b, nb, c, h, g, d = 2, 3, 5, 4, 2, 8
    q, k, v, refs = _prefill_inputs(b, nb, c, h, g, d, 11, 7, kb, seed=12)
    got = anchor.indexed_gqa(q, k, v, refs)
    r = h // g
    for bi in range(b):
        src = 0 if kb == 1 else bi
        for blk in range(nb):
            for gi in range(g):
                ref = refs[bi, blk, gi]
                kk = torch.nn.functional.pad(k[src, ref.clamp_min(0), gi], (0, 0, 0, 1))
                vv = torch.nn.functional.pad(v[src, ref.clamp_min(0), gi], (0, 0, 0, 1))
                mask = torch.nn.functional.pad(ref >= 0, (0, 1), value=True)
                qq = q[bi, blk, :, gi * r:(gi + 1) * r].permute(1, 0, 2)       # [R, C, D]
                want = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask[None, None, :])
                assert torch.allclose(got[bi, blk, :, gi * r:(gi + 1) * r], want.permute(1, 0, 2), atol=1e-12)


def test_indexed_read_of_committed_slots_is_the_decode_read():
    """One query token referencing the committed slots (dead slots as -1)
    reads exactly what the decode read returns."""
    st = workloads.anchor_state(2, 2, 64, 8, 16, dtype=torch.float64, seed=13)
    q = workloads.anchor_query(2, 4, 16, dtype=torch.float64, seed=14)
    refs = torch.arange(64).expand(2, 2, 64).masked_fill(st.positions < 0, -1)
    key = st.keys.permute(0, 2, 1, 3)                                         # [B, cap, G, D]
    val = st.values.permute(0, 2, 1, 3)
    got = anchor.indexed_gqa(q[:, None], key, val, refs[:, None])            # [B, 1, 1, H, D]
    assert torch.allclose(got[:, 0], anchor.committed_read(q, st), atol=1e-12)


def test_indexed_read_closed_forms():
    q, k, v, refs = _prefill_inputs(1, 1, 2, 1, 1, 8, 9, 4, 1, seed=15)
    refs.fill_(-1)
    assert torch.count_nonzero(anchor.indexed_gqa(q, k, v, refs)) == 0
    refs[0, 0, 0, 2] = 5
    out = anchor.indexed_gqa(q, k, v, refs)
    for t in range(2):
        logit = (q[0, 0, t, 0] @ k[0, 5, 0]).item() / math.sqrt(8)
        p = math.exp(logit) / (math.exp(logit) + 1.0)
        assert torch.allclose(out[0, 0, t, 0], p * v[0, 5, 0], atol=1e-12)


def _warm_state(b, g, cap, pc, chunk, d, steps, gen, dtype=torch.float32):
    """A state after ``steps`` decode pushes (random activity), so it carries
    committed slots, a partial pending chunk and per-row totals."""
    st = MemoryState.empty(b, g, cap, pc, d, dtype=dtype)
    for _ in range(steps):
        k = torch.randn(b, 1, g, d, generator=gen).to(dtype)
        v = torch.randn(b, 1, g, d, generator=gen).to(dtype)
        sc = torch.randn(b, 1, g, generator=gen)
        act = torch.rand(b, generator=gen) < 0.8
        anchor.commit_decode(k, v, sc, act, chunk, st)
    return st


def _token_by_token(query, key, value, scores, valid, chunk, st):
    """The decode sequence a prefill replaces: read the committed slots, then
    push (and commit on a full chunk), one token at a time."""
    b, length = query.shape[:2]
    act = torch.ones(b, length, dtype=torch.bool) if valid is None else valid
    reads = []
    for t in range(length):
        reads.append(anchor.committed_read(query[:, t:t + 1], st)[:, 0])
        anchor.commit_decode(key[:, t:t + 1], value[:, t:t + 1], scores[:, t:t + 1], act[:, t], chunk, st)
    return torch.stack(reads, 1) * act[..., None, None].to(query.dtype)


def assert_same_state(a: MemoryState, b: MemoryState):
    """Scores, positions, count and total bit-equal; key / value rows equal
    wherever a slot holds a token (a slot with no token is zero on one path
    and a copy of row 0 on the other, and is never read)."""
    assert torch.equal(a.count, b.count) and torch.equal(a.total, b.total)
    assert torch.equal(a.positions, b.positions)
    assert torch.equal(a.scores, b.scores)
    live = a.positions >= 0
    assert torch.equal(a.keys[live], b.keys[live]) and torch.equal(a.values[live], b.values[live])
    pend = torch.arange(a.pending_keys.shape[2])[None, None] < a.count[:, None, None]
    pend = pend.expand(a.pending_scores.shape)
    assert torch.equal(a.pending_keys[pend], b.pending_keys[pend])
    assert torch.equal(a.pending_values[pend], b.pending_values[pend])
    assert torch.equal(a.pending_scores[pend], b.pending_scores[pend])


@pytest.mark.parametrize("seed,cap,chunk,pc,length,warm,holes", [
    (0, 8, 4, 4, 13, 0, False),      # fresh state, several blocks, a partial tail
    (1, 8, 4, 6, 13, 7, False),      # old pending tokens open the first block; pending capacity > chunk
    (2, 6, 3, 3, 2, 5, False),       # shorter than one block
    (3, 8, 4, 4, 17, 9, True),       # invalid tokens inside the chunk
    (4, 16, 8, 8, 40, 21, True),
    (5, 4, 4, 4, 8, 3, False),       # ends exactly on a block boundary
])
def test_sequence_equals_token_by_token(seed, cap, chunk, pc, length, warm, holes):
    gen = torch.Generator().manual_seed(seed)
    b, g, h, d = 3, 2, 4, 16
    st = _warm_state(b, g, cap, pc, chunk, d, warm, gen)
    q = torch.randn(b, length, h, d, generator=gen)
    k = torch.randn(b, length, g, d, generator=gen)
    v = torch.randn(b, length, g, d, generator=gen)
    sc = torch.randn(b, length, g, generator=gen)
    sc[0, ::3] = sc[0, 1]                   # ties broken by position
    valid = (torch.rand(b, length, generator=gen) < 0.7) if holes else None
    ref_state = st.clone()
    want = _token_by_token(q, k, v, sc, valid, chunk, ref_state)
    got_state = st.clone()
    got = anchor.sequence(q, k, v, sc, valid, chunk, got_state)
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-6), (got - want).abs().max()
    assert_same_state(got_state, ref_state)
