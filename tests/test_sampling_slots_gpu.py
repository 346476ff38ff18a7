"""GPU parity of sampling and slot kernels (C-ABI path).

Bit-exact bars: counter uniforms (golden vectors of the reference), top-k
indices and values (vs torch.topk on the CPU, and a stable (value desc, index
asc) sort where values tie), sampled token ids on every row whose threshold is
not within float rounding of a CDF boundary (such rows are counted and must be
rare), bookkeeping state, slot selections, cu_seqlens and gathered rows.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sampling, slots
from yanchor_amd import inference_kernels as ik

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).parent / "golden" / "counter_sampling.npz", allow_pickle=False)


def test_counter_uniform_golden(gpu):
    ids, steps = torch.from_numpy(GOLD["ids"]).to(gpu), torch.from_numpy(GOLD["steps"]).to(gpu)
    for key in GOLD["uniform_keys"]:
        seed, stream = (int(x) for x in str(key).split("_"))
        u = ik.counter_uniform(ids, steps, seed=seed, stream=stream).cpu().numpy()
        assert np.array_equal(u, GOLD[f"uniform_{key}"])


def _ambiguous(values, idx_count, temperature, top_p, u, fused):
    """True when the draw sits within rounding of a CDF boundary (float64 check)."""
    x = values.double() / temperature
    p = torch.softmax(x, -1)
    keep = (p.cumsum(-1) - p) < top_p
    t = p * keep
    cum = t.cumsum(-1)
    thr = u * cum[-1]
    near = (cum - thr).abs().min().item() < 1e-5
    before = ((p.cumsum(-1) - p) - top_p).abs().min().item() < 1e-5
    return near or before


@pytest.mark.parametrize("case", range(6))
def test_torch_semantics_golden(gpu, case):
    logits = torch.from_numpy(GOLD["logits"])
    att, st = torch.from_numpy(GOLD["attempt_ids"]), torch.from_numpy(GOLD["row_steps"])
    t, k, p, seed = GOLD["sample_cases"][case].tolist()
    tok = ik.sample_top_k_top_p_counter(logits.to(gpu), att.to(gpu), st.to(gpu), seed=int(seed), temperature=t,
                                        top_k=int(k), top_p=p).cpu()
    want = torch.from_numpy(GOLD[f"tokens_{case}"])
    u = sampling.counter_uniform(att, st, seed=int(seed)).double()
    vals = torch.topk(logits, int(k)).values
    bad = [r for r in range(tok.shape[0]) if tok[r, 0] != want[r, 0]]
    amb = [r for r in bad if int(k) > 1 and _ambiguous(vals[r], k, t, p, u[r], False)]
    assert bad == amb, f"mismatching rows {bad}"


def _full_ambiguous(logits, t, k, p, u, vocab_order):
    """True when a full-vocabulary draw sits within float rounding of a CDF
    boundary (float64 check of the reference's definition)."""
    x = logits.double() / t
    if vocab_order:
        cum = torch.softmax(x, -1).cumsum(-1)
        return (cum - u * cum[-1]).abs().min().item() < 1e-6
    vals = torch.sort(x, descending=True).values[: (k if 0 < k < x.numel() else x.numel())]
    q = torch.softmax(vals, -1)
    before = q.cumsum(-1) - q
    keep = before < p
    kept = (q * keep).cumsum(-1)
    return ((before - p).abs().min().item() < 1e-6) or ((kept - u * kept[-1]).abs().min().item() < 1e-6)


@pytest.mark.parametrize("logits_key", ["logits", "logits_bf16"])
@pytest.mark.parametrize("case", range(7))
def test_full_vocabulary_branches_golden(gpu, logits_key, case):
    """top_k <= 0 (vocabulary order with top_p == 1; value order with a
    top_p cut) and top_k > 64 against the reference's tokens: equal on every
    row whose draw is not within rounding of a CDF boundary."""
    name = "" if logits_key == "logits" else "bf16_"
    logits = torch.from_numpy(GOLD[logits_key])
    att, st = torch.from_numpy(GOLD["attempt_ids"]), torch.from_numpy(GOLD["row_steps"])
    t, k, p, seed = GOLD["full_cases"][case].tolist()
    for dtype in ((torch.float32, torch.bfloat16) if name else (torch.float32,)):
        tok = ik.sample_top_k_top_p_counter(logits.to(dtype).to(gpu), att.to(gpu), st.to(gpu), seed=int(seed),
                                            temperature=t, top_k=int(k), top_p=p).cpu()
        want = torch.from_numpy(GOLD[f"full_{name}tokens_{case}"])
        u = sampling.counter_uniform(att, st, seed=int(seed)).double()
        bad = [r for r in range(tok.shape[0]) if tok[r, 0] != want[r, 0]]
        vocab_order = int(k) <= 0 and p == 1.0
        ties = [r for r in bad if _drawn_rank_ties(logits[r], t, int(k), p, u[r].item())]
        amb = [r for r in bad if r in ties or _full_ambiguous(logits[r], t, int(k), p, u[r].item(), vocab_order)]
        assert bad == amb, f"mismatching rows {bad} ({dtype})"
        # inside a tie group the drawn score is the reference's, only the index
        # among equal scores is torch.topk's unpinned order
        assert all(logits[r, tok[r, 0]] == logits[r, want[r, 0]] for r in ties)


@pytest.mark.parametrize("t,k,p", [(0.6, 0, 1.0), (0.6, 0, 0.95), (1.0, 200, 0.9), (0.8, 151936, 0.99)])
def test_full_vocabulary_branches_at_decode_shape(gpu, t, k, p):
    """B = 128 rows of the 151936-token vocabulary, bf16 logits with the
    presence penalty: the oracle's tokens (torch on the host) on every row
    away from a CDF boundary; repeated calls give the same tokens."""
    b, v = 128, 151936
    g = torch.Generator().manual_seed(int(t * 100) + k)
    logits = (torch.randn(b, v, generator=g) * 3).to(torch.bfloat16)
    seen = torch.rand(b, v, generator=g) < 0.001
    att, st = torch.arange(b) * 7 + 1, torch.randint(0, 4000, (b,), generator=g)
    d = logits.to(gpu)
    tok = ik.topk_sample(d, att.to(gpu), st.to(gpu), seed=20260923, temperature=t, top_k=k, top_p=p,
                         mode=ik.SAMPLE_TORCH, seen=seen.to(gpu), presence_penalty=1.5).cpu()
    again = ik.topk_sample(d, att.to(gpu), st.to(gpu), seed=20260923, temperature=t, top_k=k, top_p=p,
                           mode=ik.SAMPLE_TORCH, seen=seen.to(gpu), presence_penalty=1.5).cpu()
    assert torch.equal(tok, again)
    scores = sampling.presence_penalty(logits.float(), seen, 1.5)
    want = sampling.sample_top_k_top_p_counter(scores, att, st, seed=20260923, temperature=t, top_k=k, top_p=p)
    u = sampling.counter_uniform(att, st, seed=20260923).double()
    bad = [r for r in range(b) if tok[r, 0] != want[r, 0]]
    # bf16 logits tie exactly: rows whose kept set ends inside a tie group may
    # order the ties differently from torch.topk (tie order is unpinned there)
    ties = [r for r in bad if _drawn_rank_ties(scores[r], t, k, p, u[r].item())]
    amb = [r for r in bad if r in ties or _full_ambiguous(scores[r], t, k, p, u[r].item(), k <= 0 and p == 1.0)]
    print(f"t={t} k={k} p={p}: {len(bad)} mismatching rows: {len(ties)} inside a tie group, "
          f"{len(amb) - len(ties)} at a CDF boundary", flush=True)
    assert bad == amb, f"mismatching rows {bad}"
    assert len(amb) - len(ties) <= 2                     # boundary cases are rare
    # bf16 logits tie exactly: inside a tie group the drawn score is the
    # reference's; which of the equal scores comes first is torch.topk's
    # unpinned tie order (the kernel takes the lowest index)
    assert all(scores[r, tok[r, 0]] == scores[r, want[r, 0]] for r in ties)


def _drawn_rank_ties(scores, t, k, p, u):
    """In value order, the drawn rank's value equals a neighbour's: which of
    the tied indices sits at that rank is torch.topk's unpinned tie order
    (the kernel puts the lower index first)."""
    if k <= 0 and p == 1.0:
        return False
    vals = torch.sort(scores.double() / t, descending=True).values
    vals = vals[: (k if 0 < k < vals.numel() else vals.numel())]
    q = torch.softmax(vals, -1)
    kept = (q * ((q.cumsum(-1) - q) < p)).cumsum(-1)
    r = int(torch.searchsorted(kept, u * kept[-1]))
    return bool((r > 0 and vals[r] == vals[r - 1]) or (r + 1 < vals.numel() and vals[r] == vals[r + 1]))


@pytest.mark.parametrize("b,v,k,dtype", [(8, 1000, 20, torch.float32), (128, 151936, 20, torch.float32),
                                         (128, 151936, 20, torch.bfloat16), (4, 151936, 32, torch.bfloat16),
                                         (4, 151936, 33, torch.float32), (5, 70000, 64, torch.float32),
                                         (3, 37, 7, torch.float32), (4, 4096, 1, torch.bfloat16)])
def test_topk_matches_torch(gpu, b, v, k, dtype):
    g = torch.Generator().manual_seed(b * v + k)
    logits = (torch.randn(b, v, generator=g) * 4).to(dtype)
    tok, vals, idx = ik.topk_sample(logits.to(gpu), torch.arange(b).to(gpu), 0, seed=1, temperature=0.6,
                                    top_k=k, top_p=0.95, mode=ik.SAMPLE_FUSED, return_topk=True)
    rv, ri = torch.topk(logits.float(), k)       # bf16 ties: torch.topk keeps no index order, so compare in fp32
    if dtype == torch.float32:
        assert torch.equal(idx.cpu(), ri) and torch.equal(vals.cpu(), rv)
    else:
        order = torch.sort(-logits.float() * 1.0, dim=-1, stable=True).indices[:, :k]
        assert torch.equal(idx.cpu(), order) and torch.equal(vals.cpu(), torch.gather(logits.float(), 1, order))


def _topk_two_kernels(logits, seen, penalty, k):
    """Top-k (values, indices) of bf16 rows on the 16384-element bf16 kernel
    and of the same values as float32 on the 8192-element kernel."""
    dev, b = logits.device, logits.shape[0]
    kw = dict(seed=1, temperature=1.0, top_k=k, top_p=1.0, mode=ik.SAMPLE_FUSED, return_topk=True, seen=seen,
              presence_penalty=penalty)
    _, v1, i1 = ik.topk_sample(logits, torch.arange(b, device=dev), 0, **kw)
    _, v2, i2 = ik.topk_sample(logits.float(), torch.arange(b, device=dev), 0, **kw)
    return v1.cpu(), i1.cpu(), v2.cpu(), i2.cpu()


def _stable_topk(adjusted, k):
    order = torch.sort(-adjusted, dim=-1, stable=True).indices[:, :k]
    return torch.gather(adjusted, 1, order), order


@pytest.mark.parametrize("v", [151936, 32768, 20000, 40])
@pytest.mark.parametrize("k", [1, 7, 20, 32])
@pytest.mark.parametrize("density,penalty", [(0.0, 0.0), (0.01, 1.5), (0.3, 1.5), (0.3, -0.5)])
def test_bf16_topk_kernel(gpu, v, k, density, penalty):
    """bf16 rows with top_k <= 32 (the 16384-element kernel; the last segment
    partial except at 32768, fewer than k thread maxima at V = 40): the same
    lists as the float32 kernel on the same values, and the stable (value
    desc, index asc) top k of the penalised scores."""
    if k > v:
        pytest.skip("k above the vocabulary")
    b = 6
    g = torch.Generator().manual_seed(v + k + int(density * 100))
    logits = (torch.randn(b, v, generator=g) * 3).to(torch.bfloat16)
    seen = torch.rand(b, v, generator=g) < density
    v1, i1, v2, i2 = _topk_two_kernels(logits.to(gpu), seen.to(gpu), penalty, k)
    assert torch.equal(i1, i2) and torch.equal(v1, v2)
    rv, ri = _stable_topk(logits.float() - penalty * seen.float(), k)
    assert torch.equal(i1, ri) and torch.equal(v1, rv)


@pytest.mark.parametrize("k", [1, 20, 32])
def test_bf16_topk_kernel_ties_and_specials(gpu, k):
    """Rows built against the threshold: every value equal (with and without
    seen elements), +-0 mixed, a few large values over a sea of equal ones,
    the largest elements all seen (their penalised values still on top for
    some rows), and equal maxima in more threads than the list holds."""
    v = 40000
    rows, seens = [], []
    z = torch.zeros(v)
    rows.append(z.clone()); seens.append(torch.zeros(v, dtype=torch.bool))
    s = torch.zeros(v, dtype=torch.bool); s[::3] = True
    rows.append(z.clone()); seens.append(s)
    r = torch.zeros(v); r[1::2] = -0.0; r[17000] = 0.5; r[39999] = 0.5
    rows.append(r); seens.append(torch.zeros(v, dtype=torch.bool))
    r = torch.full((v,), 1.25); r[[5, 900, 20000, 33333]] = 4.0
    rows.append(r); seens.append(torch.zeros(v, dtype=torch.bool))
    g = torch.Generator().manual_seed(3)
    r = torch.randn(v, generator=g)
    top = torch.topk(r, 64).indices
    s = torch.zeros(v, dtype=torch.bool); s[top] = True
    rows.append(r); seens.append(s)
    r = torch.randn(v, generator=g).clamp(max=1.0)
    r[torch.randperm(v, generator=g)[:500]] = 2.0         # 500 equal maxima spread over the threads
    rows.append(r); seens.append(torch.zeros(v, dtype=torch.bool))
    logits = torch.stack(rows).to(torch.bfloat16)
    seen = torch.stack(seens)
    v1, i1, v2, i2 = _topk_two_kernels(logits.to(gpu), seen.to(gpu), 1.5, k)
    assert torch.equal(i1, i2) and torch.equal(v1, v2)
    rv, ri = _stable_topk(logits.float() - 1.5 * seen.float(), k)
    assert torch.equal(i1, ri) and torch.equal(v1, rv)


def test_bf16_topk_kernel_nan_and_seen_bytes(gpu):
    """NaN logits (which the float maxima skip) send the segment through the
    exact element keys: the same lists as the float32 kernel (positive NaN
    above every number, negative NaN below).  Seen bytes other than 0 / 1
    count as seen."""
    b, v, k = 4, 70000, 20
    g = torch.Generator().manual_seed(8)
    logits = (torch.randn(b, v, generator=g) * 2).to(torch.bfloat16)
    logits[0, 123] = float("nan")
    logits[1, 50000] = -float("nan")
    logits[2, [7, 40000]] = float("nan")
    raw = (torch.rand(b, v, generator=g) < 0.2).to(torch.uint8) * torch.randint(1, 256, (b, v), generator=g,
                                                                                dtype=torch.uint8)
    seen = raw.view(torch.bool)                          # nonzero bytes, not only 1
    v1, i1, v2, i2 = _topk_two_kernels(logits.to(gpu), seen.to(gpu), 1.5, k)
    assert torch.equal(i1, i2) and torch.equal(v1.isnan(), v2.isnan())
    assert torch.equal(v1[~v1.isnan()], v2[~v2.isnan()])
    rv, ri = _stable_topk(logits[3:].float() - 1.5 * (raw[3:] != 0).float(), k)   # the row without NaN
    assert torch.equal(i1[3:], ri) and torch.equal(v1[3:], rv)


@pytest.mark.parametrize("k", [20, 32, 33])
def test_topk_all_equal_segments(gpu, k):
    """Every element ties: the lowest k indices, for the wave threshold (k <=
    32) at its worst candidate count and for the exact one above it."""
    logits = torch.zeros(3, 151936, dtype=torch.bfloat16)
    logits[1, 50000:] = 1.0
    _, vals, idx = ik.topk_sample(logits.to(gpu), torch.arange(3).to(gpu), 0, seed=1, temperature=1.0, top_k=k,
                                  top_p=1.0, mode=ik.SAMPLE_FUSED, return_topk=True)
    assert idx[0].cpu().tolist() == list(range(k)) and idx[2].cpu().tolist() == list(range(k))
    assert idx[1].cpu().tolist() == list(range(50000, 50000 + k))


def test_topk_ties_lower_index_first(gpu):
    logits = torch.zeros(3, 5000)
    logits[0, ::7] = 1.0          # many equal maxima
    logits[1] = -0.0              # all -0.0 == +0.0
    logits[2, 100:200] = 2.5
    _, vals, idx = ik.topk_sample(logits.to(gpu), torch.arange(3).to(gpu), 0, seed=1, temperature=1.0, top_k=16,
                                  top_p=1.0, mode=ik.SAMPLE_FUSED, return_topk=True)
    for r in range(3):
        order = sorted(range(5000), key=lambda i: (-logits[r, i].item(), i))[:16]
        assert idx[r].cpu().tolist() == order


@pytest.mark.parametrize("temperature,top_p", [(0.6, 0.95), (1.0, 0.5), (1.7, 1.0)])
def test_fused_semantics_vs_oracle(gpu, temperature, top_p):
    b, v = 128, 151936
    g = torch.Generator().manual_seed(17)
    logits = torch.randn(b, v, generator=g) * 3
    att = torch.randint(0, 10**9, (b,), generator=g)
    steps = torch.randint(0, 10**5, (b,), generator=g)
    tok = ik.sample_top20_counter(logits.to(gpu), att.to(gpu), steps.to(gpu), seed=20260923,
                                  temperature=temperature, top_p=top_p).cpu()
    vals, idx = torch.topk(logits, 20)
    want = sampling.top20_counter_sample(vals / temperature, idx, att, steps, seed=20260923, top_p=top_p)
    u = torch.tensor([(sampling.counter_word(int(a), int(s), 20260923) + 0.5) / 2**32 for a, s in zip(att, steps)])
    bad = [r for r in range(b) if tok[r, 0] != want[r, 0]]
    amb = [r for r in bad if _ambiguous(vals[r], 20, temperature, top_p, u[r], True)]
    assert bad == amb and len(amb) <= 2, f"mismatching rows {bad}"


def test_fused_presence_penalty(gpu):
    b, v = 16, 20000
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(b, v, generator=g) * 3
    seen = torch.rand(b, v, generator=g) < 0.3
    att, steps = torch.arange(b), torch.full((b,), 9)
    tok = ik.sample_top20_counter(logits.to(gpu), att.to(gpu), steps.to(gpu), seed=3, temperature=0.6,
                                  top_p=0.95, seen=seen.to(gpu), presence_penalty=1.5).cpu()
    adjusted = sampling.presence_penalty(logits, seen, 1.5)
    vals, idx = torch.topk(adjusted, 20)
    want = sampling.top20_counter_sample(vals / 0.6, idx, att, steps, seed=3, top_p=0.95)
    assert (tok == want).all()
    # the standalone in-place kernel gives the same adjusted scores
    sc = logits.clone().to(gpu)
    ik._apply_dense_presence_penalty_(sc, seen.to(gpu), 1.5)
    assert torch.equal(sc.cpu(), adjusted)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_topk_elementwise_path_with_penalty(gpu, dtype):
    """A vocabulary that is not a multiple of the 16-byte run takes the
    element-by-element loads (three segments, the last partial) with the seen
    mask's penalty applied: the top k of the penalised scores, lower index
    first on ties."""
    b, v, k = 6, 20001, 24
    g = torch.Generator().manual_seed(31)
    logits = (torch.randn(b, v, generator=g) * 2).to(dtype)
    seen = torch.rand(b, v, generator=g) < 0.2
    _, vals, idx = ik.topk_sample(logits.to(gpu), torch.arange(b).to(gpu), 0, seed=1, temperature=1.0, top_k=k,
                                  top_p=1.0, mode=ik.SAMPLE_FUSED, return_topk=True, seen=seen.to(gpu),
                                  presence_penalty=1.5)
    adjusted = logits.float() - 1.5 * seen.float()
    order = torch.sort(-adjusted, dim=-1, stable=True).indices[:, :k]
    assert torch.equal(idx.cpu(), order) and torch.equal(vals.cpu(), torch.gather(adjusted, 1, order))


def test_strided_rows(gpu):
    logits = torch.randn(6, 3000)
    view = logits.to(gpu)[:, :2500]
    _, vals, idx = ik.topk_sample(view, torch.arange(6).to(gpu), 0, seed=1, temperature=1.0, top_k=20, top_p=1.0,
                                  mode=ik.SAMPLE_TORCH, return_topk=True)
    rv, ri = torch.topk(logits[:, :2500], 20)
    assert torch.equal(idx.cpu(), ri)


def _scenario(seed, slots_n=96, attempts=300, width=40, vocab=1000):
    g = torch.Generator().manual_seed(seed)
    return dict(
        sampled=torch.randint(0, vocab, (slots_n, 1), generator=g),
        storage=torch.full((attempts + slots_n, width + 1), 7, dtype=torch.int32),
        dense_seen=torch.rand(slots_n, vocab, generator=g) < 0.05,
        generated_lengths=torch.randint(0, 3, (attempts + slots_n,), generator=g),
        finished_by_eos=torch.zeros(attempts + slots_n, dtype=torch.bool),
        finished=torch.rand(slots_n, generator=g) < 0.2,
        slot_rows=torch.where(torch.rand(slots_n, generator=g) < 0.85,
                              torch.randperm(attempts, generator=g)[:slots_n], torch.tensor(-1)),
        sink_rows=attempts + torch.arange(slots_n),
        slot_caps=torch.randint(2, width, (slots_n,), generator=g),
        row_steps=torch.randint(1, 3, (slots_n,), generator=g),
        row_positions=torch.randint(5, 50, (slots_n,), generator=g),
        decode_ids=torch.zeros(slots_n, 1, dtype=torch.long),
        useful=torch.zeros((), dtype=torch.long),
    ), g


def test_bookkeeping_bit_exact(gpu):
    cpu, g = _scenario(1)
    dev = {k: v.to(gpu) for k, v in cpu.items()}
    kw = dict(maximum_new_tokens=40, pad_token_id=7, eos_token_ids=(3, 4))
    for step in range(30):
        tok = torch.randint(0, 1000, (96, 1), generator=g)
        tok[tok % 97 == 0] = 3  # some eos
        cpu["sampled"], dev["sampled"] = tok.clone(), tok.to(gpu)
        slots.decode_state_update(*cpu.values(), **kw)
        ik._update_fixed_decode_state_(*dev.values(), **kw)
        torch.cuda.synchronize()
        for k in cpu:
            assert torch.equal(dev[k].cpu(), cpu[k]), f"{k} differs at step {step}"


@pytest.mark.parametrize("n", [0, 1, 7, 1024, 1500, 5000])
def test_selection_and_cu_seqlens(gpu, n):
    g = torch.Generator().manual_seed(n)
    fin = torch.rand(n, generator=g) < 0.4
    rows = torch.where(torch.rand(n, generator=g) < 0.8, torch.arange(n), torch.tensor(-1))
    keep = ik.compaction_keep(fin.to(gpu), rows.to(gpu)).cpu().tolist()
    assert keep == slots.compaction_keep(fin, rows)
    assert ik.refill_targets(fin.to(gpu)).cpu().tolist() == slots.refill_targets(fin)
    lengths = torch.randint(0, 9000, (n,), generator=g)
    for dt in (torch.int32, torch.int64):
        cu = ik.cu_seqlens(lengths.to(dt).to(gpu)).cpu().tolist()
        assert cu == slots.cu_seqlens(lengths.tolist())


def test_gather_rows(gpu):
    g = torch.Generator().manual_seed(2)
    src = [torch.randn(10, 32, 128, 128, generator=g), torch.randint(0, 100, (10,), generator=g),
           torch.randn(10, 3, 5, generator=g).to(torch.bfloat16), torch.rand(10, generator=g) < 0.5]
    dst = [torch.zeros_like(t) for t in src]
    si = torch.tensor([9, 0, 3, 3])
    di = torch.tensor([1, 2, 5, 8])
    ds = [t.to(gpu) for t in src]
    dd = [t.to(gpu) for t in dst]
    ik.gather_rows(list(zip(ds, dd)), si.to(gpu), di.to(gpu))
    for s, d, outd in zip(src, dst, dd):
        d.index_copy_(0, di, s.index_select(0, si))
        assert torch.equal(outd.cpu(), d)
