"""GPU parity of the anchor-memory kernels (C-ABI path) with the oracle.

* read: bf16 output within 2e-2 Frobenius relative error of the float64 oracle
  (observed ~2e-3); fp32 within 1e-3;
* commit: bit-exact state (keys, values, scores, positions, pending, count,
  total) after every step of multi-chunk decode sequences, with forced score
  ties, -0.0, inactive rows and slot indirection;
* prefill read (indexed_gqa): bf16 / fp16 output within 1e-2 of the float64
  oracle, with dead and out-of-range references, ragged tiles (CAP and
  C * H/G not multiples of 64), a shared key batch and int32 / int64
  references.
"""
import math
from dataclasses import fields

import pytest
import torch

from oracle import anchor as ref
from yanchor_amd import independent_memory as im
from yanchor_amd import workloads

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _to(st, device):
    return im.IndependentMemoryState(*(getattr(st, f.name).to(device) for f in fields(st)))


def _oracle_state(st):
    return ref.MemoryState(*(getattr(st, f.name).cpu().clone() for f in fields(st)))


def _assert_state_equal(got, want):
    for f in fields(want):
        a, b = getattr(got, f.name).cpu(), getattr(want, f.name).cpu()
        assert torch.equal(a, b), f"state field {f.name} differs"


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-3)])
@pytest.mark.parametrize("r", [1, 2, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_read_matches_oracle(gpu, dtype, tol, r, d):
    st = workloads.anchor_state(6, 2, 256, 64, d, dtype=dtype, seed=r * 7 + d)
    q = workloads.anchor_query(6, 2 * r, d, dtype=dtype, seed=r + d)
    want = ref.committed_read(q, st)
    got = im.committed_gqa(q.to(gpu), _to(st, gpu))
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == q.shape
    assert rel_err(got, want) <= tol, rel_err(got, want)


@pytest.mark.parametrize("cap", [16, 48, 96])
@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-3)])
def test_read_small_capacities(gpu, cap, dtype, tol):
    """Capacities that are not multiples of the 32-slot block (16-slot
    blocks) or give an odd block count."""
    st = workloads.anchor_state(5, 2, cap, 64, 128, dtype=dtype, seed=cap + 3)
    q = workloads.anchor_query(5, 8, 128, dtype=dtype, seed=cap + 4)
    got = im.committed_gqa(q.to(gpu), _to(st, gpu))
    want = ref.committed_read(q, st)
    assert rel_err(got, want) <= tol, rel_err(got, want)


def test_commit_top16_of_chunk64(gpu):
    """The long-horizon setting: 16 committed slots, commit chunk 64 (the best
    16 of 80 candidates kept)."""
    st = workloads.anchor_state(4, 8, 16, 64, 128, seed=31, fill_pending=50)
    assert _drive(gpu, st, 40, 64, seed=32, p_active=0.95) >= 4


def test_read_decode_config(gpu):
    """64 rows x 32 groups x 256 slots x 128 dims bf16, slots live with p = 0.7."""
    st = workloads.anchor_state(64, 32, 256, 64, 128, seed=workloads.SEED0 + 1)
    q = workloads.anchor_query(64, 32, 128)
    got = im.committed_gqa(q.to(gpu), _to(st, gpu))
    want = ref.committed_read(q, st)
    assert rel_err(got, want) <= 2e-2


def test_read_empty_and_indirect(gpu):
    st = workloads.anchor_state(4, 2, 128, 16, 128, seed=3)
    st.positions[1] = -1  # row 1 has no live slot: output 0 (only the sink)
    q = workloads.anchor_query(3, 2, 128, seed=4)
    idx = torch.tensor([1, -1, 2], dtype=torch.int32)
    got = im.committed_gqa(q.to(gpu), _to(st, gpu), idx.to(gpu)).cpu()
    assert torch.count_nonzero(got[0]) == 0 and torch.count_nonzero(got[1]) == 0
    want = ref.committed_read(q, st, idx)
    assert rel_err(got[2], want[2]) <= 2e-2


def _drive(gpu, st, steps, chunk, seed, indices=None, tie_scores=False, p_active=0.9, fused_kv=False):
    """Run `steps` decode pushes on GPU and oracle, comparing after each.
    fused_kv: the device key / value are the two halves of one [B, 1, 2G, D]
    row (batch rows 2 G D elements apart, as a fused k/v projection)."""
    b_rows = st.count.shape[0] if indices is None else indices.shape[0]
    g, d = st.keys.shape[1], st.keys.shape[3]
    gen = torch.Generator().manual_seed(seed)
    dev_state = _to(st, gpu)
    o_state = _oracle_state(st)
    dev_idx = None if indices is None else indices.to(gpu)
    commits = 0
    for step in range(steps):
        key = torch.randn(b_rows, 1, g, d, generator=gen).to(st.keys.dtype)
        val = torch.randn(b_rows, 1, g, d, generator=gen).to(st.keys.dtype)
        sc = torch.randn(b_rows, 1, g, generator=gen)
        if tie_scores:
            sc = sc.round()
            sc[sc == 0] = torch.where(torch.rand(int((sc == 0).sum()), generator=gen) < 0.5,
                                      torch.tensor(0.0), torch.tensor(-0.0))
        active = torch.rand(b_rows, generator=gen) < p_active
        will = [(int(o_state.count[i if indices is None else int(indices[i])]) + 1 == chunk) and bool(active[i])
                and (indices is None or int(indices[i]) >= 0) for i in range(b_rows)]
        commits += sum(will)
        if fused_kv:
            kv = torch.cat((key, val), 2).to(gpu)
            dk, dv = kv[:, :, :g], kv[:, :, g:]
            assert dk.stride(0) == 2 * g * d and not dv.is_contiguous()
        else:
            dk, dv = key.to(gpu), val.to(gpu)
        im.commit_decode(dk, dv, sc.to(gpu), active.to(gpu), chunk, dev_state, dev_idx)
        ref.commit_decode(key, val, sc, active, chunk, o_state, indices)
        torch.cuda.synchronize()
        _assert_state_equal(dev_state, o_state)
    return commits


def test_commit_bit_exact_small_chunks(gpu):
    st = workloads.anchor_state(3, 2, 64, 8, 128, seed=21, fill_pending=0)
    assert _drive(gpu, st, 40, 8, seed=22) > 5


def test_commit_bit_exact_with_ties_and_indices(gpu):
    st = workloads.anchor_state(5, 3, 64, 16, 64, seed=23, fill_pending=5)
    st.scores.copy_(torch.where(st.positions >= 0, st.scores.round(), st.scores))
    idx = torch.tensor([4, 0, -1, 2], dtype=torch.int32)
    assert _drive(gpu, st, 30, 12, seed=24, indices=idx, tie_scores=True) > 2


def test_commit_decode_config_chunk64(gpu):
    """256 committed slots, commit chunk 64, 128-d bf16 (the decode layout)."""
    st = workloads.anchor_state(4, 4, 256, 64, 128, seed=25, fill_pending=60)
    assert _drive(gpu, st, 10, 64, seed=26, p_active=1.0) >= 4


def test_commit_fused_kv_rows(gpu):
    """Key / value read in place from the halves of a fused projection row."""
    st = workloads.anchor_state(4, 8, 64, 8, 128, seed=29, fill_pending=3)
    idx = torch.tensor([3, 1, -1, 0], dtype=torch.int32)
    assert _drive(gpu, st, 24, 8, seed=30, indices=idx, fused_kv=True) > 2


def test_commit_fp32_rows(gpu):
    st = workloads.anchor_state(2, 2, 64, 4, 64, dtype=torch.float32, seed=27)
    assert _drive(gpu, st, 12, 4, seed=28) > 2


def _prefill(b, nb, c, h, g, s, cap, kb, dtype, ref_dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, nb, c, h, 128, generator=gen).to(dtype)
    k = torch.randn(kb, s, g, 128, generator=gen).to(dtype)
    v = torch.randn(kb, s, g, 128, generator=gen).to(dtype)
    refs = torch.randint(0, s, (b, nb, g, cap), generator=gen)
    refs[torch.rand(b, nb, g, cap, generator=gen) < 0.3] = -1
    refs[..., -1] = s + 3                     # out of range: counts as none
    return q, k, v, refs.to(ref_dtype)


@pytest.mark.parametrize("b,nb,c,h,g,s,cap,kb", [(2, 3, 64, 8, 2, 300, 256, 2), (1, 2, 10, 8, 2, 50, 100, 1),
                                                 (3, 1, 64, 4, 4, 700, 64, 3), (2, 2, 33, 16, 2, 129, 130, 1)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ref_dtype", [torch.int64, torch.int32])
def test_indexed_read_matches_oracle(gpu, b, nb, c, h, g, s, cap, kb, dtype, ref_dtype):
    q, k, v, refs = _prefill(b, nb, c, h, g, s, cap, kb, dtype, ref_dtype, seed=b * 1000 + c + cap)
    got = im.indexed_gqa(q.to(gpu), k.to(gpu), v.to(gpu), refs.to(gpu))
    torch.cuda.synchronize()
    want = ref.indexed_gqa(q, k, v, refs)
    assert got.dtype == dtype and got.shape == q.shape
    assert rel_err(got, want) <= 1e-2, rel_err(got, want)


def test_indexed_read_no_references(gpu):
    q, k, v, refs = _prefill(1, 2, 64, 4, 2, 20, 64, 1, torch.bfloat16, torch.int64, seed=3)
    refs.fill_(-1)
    got = im.indexed_gqa(q.to(gpu), k.to(gpu), v.to(gpu), refs.to(gpu))
    assert torch.count_nonzero(got) == 0


@pytest.mark.parametrize("b,g,h,cap,pc,chunk,length,fill,holes,empty", [
    (4, 2, 8, 64, 8, 8, 37, 3, False, False),     # unsorted committed slots, old pending tokens, ragged tail
    (4, 2, 8, 64, 10, 8, 37, 5, True, False),     # invalid tokens; pending capacity > chunk
    (3, 2, 4, 64, 8, 8, 5, 2, False, False),      # no block completes: the committed slots are only re-ranked
    (2, 8, 32, 256, 64, 64, 300, 10, False, False),   # the decode layout: 256 slots, chunk 64, 8 groups
    (5, 8, 32, 256, 64, 64, 128, 0, False, True),     # fresh state (a prompt prefill), whole blocks only
])
def test_sequence_matches_oracle(gpu, b, g, h, cap, pc, chunk, length, fill, holes, empty):
    """Prefill continuation on the GPU against the oracle's restatement of
    _sequence: the state bit-exact (memory kept in rank order, pending tail,
    count, total, zeroed dead slots), the read within 1e-2 of the float64
    oracle."""
    d = 128
    seed = b * 100 + length
    if empty:
        st = im.IndependentMemoryState.empty(b, g, cap, pc, d, "cpu", torch.bfloat16)
    else:
        st = workloads.anchor_state(b, g, cap, pc, d, seed=seed, fill_pending=fill)
    gen = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(b, length, h, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, length, g, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, length, g, d, generator=gen).to(torch.bfloat16)
    sc = torch.randn(b, length, g, generator=gen)
    sc[:, 1::4] = sc[:, ::4][:, : sc[:, 1::4].shape[1]]      # score ties, broken by position
    valid = (torch.rand(b, length, generator=gen) < 0.75) if holes else None
    o_state = _oracle_state(st)
    want = ref.sequence(q, k, v, sc, valid, chunk, o_state)
    dev_state = _to(st, gpu)
    got = im.sequence(q.to(gpu), k.to(gpu), v.to(gpu), sc.to(gpu), None if valid is None else valid.to(gpu), chunk,
                      dev_state)
    torch.cuda.synchronize()
    assert got.shape == q.shape and got.dtype == q.dtype
    _assert_state_equal(dev_state, o_state)
    assert rel_err(got, want) <= 1e-2, rel_err(got, want)
    if valid is not None:
        assert not got.cpu()[~valid].any()


def test_sequence_then_decode_continues(gpu):
    """A prefill continuation followed by decode pushes leaves the same state
    as the oracle doing the same, so the two paths hand over cleanly."""
    b, g, h, cap, pc, chunk, d = 3, 2, 8, 64, 8, 8, 128
    st = workloads.anchor_state(b, g, cap, pc, d, seed=41, fill_pending=6)
    gen = torch.Generator().manual_seed(42)
    q = torch.randn(b, 21, h, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, 21, g, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, 21, g, d, generator=gen).to(torch.bfloat16)
    sc = torch.randn(b, 21, g, generator=gen)
    o_state = _oracle_state(st)
    ref.sequence(q, k, v, sc, None, chunk, o_state)
    dev_state = _to(st, gpu)
    im.sequence(q.to(gpu), k.to(gpu), v.to(gpu), sc.to(gpu), None, chunk, dev_state)
    torch.cuda.synchronize()
    _assert_state_equal(dev_state, o_state)
    _drive_from(gpu, dev_state, o_state, 12, chunk, seed=43)


def _drive_from(gpu, dev_state, o_state, steps, chunk, seed):
    b, g, d = o_state.count.shape[0], o_state.keys.shape[1], o_state.keys.shape[3]
    gen = torch.Generator().manual_seed(seed)
    for _ in range(steps):
        key = torch.randn(b, 1, g, d, generator=gen).to(o_state.keys.dtype)
        val = torch.randn(b, 1, g, d, generator=gen).to(o_state.keys.dtype)
        sc = torch.randn(b, 1, g, generator=gen)
        active = torch.ones(b, dtype=torch.bool)
        im.commit_decode(key.to(gpu), val.to(gpu), sc.to(gpu), active.to(gpu), chunk, dev_state)
        ref.commit_decode(key, val, sc, active, chunk, o_state)
        torch.cuda.synchronize()
        live = o_state.positions >= 0
        for name in ("scores", "positions", "count", "total"):
            assert torch.equal(getattr(dev_state, name).cpu(), getattr(o_state, name)), name
        assert torch.equal(dev_state.keys.cpu()[live], o_state.keys[live])


def test_read_gated_equals_read_then_gates(gpu):
    """The fused gating epilogue is the torch gating of the plain read, bit for
    bit (every product rounded to bf16 the same way)."""
    from yanchor_amd.runtime import gate_read
    st = _to(workloads.anchor_state(6, 2, 256, 64, 128, seed=70), gpu)
    q = workloads.anchor_query(6, 8, 128, seed=71).to(gpu)
    valid = torch.tensor([True, False, True, True, False, True], device=gpu)
    hg = torch.rand(6, 8, device=gpu) * 2
    plain = im.committed_gqa(q, st)
    got = im.committed_gqa_gated(q, st, None, valid, hg)
    assert torch.equal(got, gate_read(plain, valid, hg))
    assert torch.equal(im.committed_gqa_gated(q, st, None, valid, None), gate_read(plain, valid))


def test_window_attend_gated(gpu):
    from yanchor_amd.runtime import gate_read
    b, g, win, d, h = 4, 2, 128, 128, 8
    gen = torch.Generator(device=gpu).manual_seed(80)
    keys = torch.randn(b, g, win, d, device=gpu, generator=gen).to(torch.bfloat16)
    vals = torch.randn(b, g, win, d, device=gpu, generator=gen).to(torch.bfloat16)
    pos = torch.where(torch.rand(b, g, win, device=gpu, generator=gen) < 0.8,
                      torch.arange(win, device=gpu, dtype=torch.int32), torch.tensor(-1, device=gpu, dtype=torch.int32))
    q = torch.randn(b, 1, h, d, device=gpu, generator=gen).to(torch.bfloat16)
    qg = torch.randn(b, h, 2 * d, device=gpu, generator=gen).to(torch.bfloat16)
    gate = qg[..., d:]                                       # strided, as in the fused q | gate projection
    got = im.ring_decode_attention(q, keys, vals, pos, gate=gate)
    want = gate_read(im.ring_decode_attention(q, keys, vals, pos), gate=gate)
    assert got.shape == want.shape
    diff = (got.float() - want.float()).abs()
    assert (diff <= want.float().abs() * 2.0 ** -7 * 1.0001 + 1e-30).all()
    assert (got != want).float().mean().item() <= 0.01
