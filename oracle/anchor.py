"""Fixed-slot anchor memory on the CPU (oracle; test infrastructure only).

Restates, from the reference:

* ``MemoryState``        IndependentMemoryState, modeling_yanchor.py:80-120
* ``select_topk``        modeling_yanchor.py:51-60
* ``merge_topk``         modeling_yanchor.py:62-63
* ``exclusive_prefix_topk``  modeling_yanchor.py:65-78 (brute-force form)
* ``indexed_gqa``        the prefill read over referenced rows,
                         modeling_yanchor.py:22-42, independent_memory.py:6-45
* ``committed_read``     the decode read, modeling_yanchor.py:283-290, with the
                         slot indirection and zero-logit sink of
                         runtime/model/independent_memory.py:47-88, 177-188
* ``commit_decode``      the decode push + Top-K commit, modeling_yanchor.py:
                         291-312, with the slot indirection of
                         runtime/model/independent_memory.py:90-175, 190-201
* ``sequence``           the prefill read / write continuing a state,
                         IndependentGQAMemory._sequence, modeling_yanchor.py:
                         178-275 (given every token's key / value)
* ``committed_read_batched`` / ``commit_decode_batched``  the same decode read
                         and commit over the whole batch at once, the
                         reference's torch branch of _decode
                         (modeling_yanchor.py:283-313): the host CPU baseline's
                         form, equal to the per-row restatements above

Ordering contract of every Top-K here: candidates are ordered by
(score descending, position ascending with invalid last, candidate index
ascending); -0.0 ranks equal to +0.0.  That is the composition of the two
stable sorts in select_topk (position first, then score) and the two packed
u64 sorts of _push_select (independent_memory.py:115-128).

Pins (tests/test_oracle_anchor.py): the tensor ``select_topk`` agrees with a
brute-force ``sorted()`` on random inputs with forced ties, -0.0 and invalid
slots; the read equals a softmax over [logits, 0] computed independently and
reduces to closed forms for zero / one valid slot; ``indexed_gqa`` equals an
SDPA over the gathered rows plus a zero row, and equals ``committed_read`` when
a single token references the committed slots; ``exclusive_prefix_topk``
is checked against the O(n^2) definition "Top-K of every earlier block";
``sequence`` (prefix Top-K of blocks, merged with the committed slots, one
indexed read per block) equals the token-by-token committed_read /
commit_decode sequence it replaces -- reads, and the state it leaves; the
batched read and commit equal the per-row ones (the state bit for bit) over
staggered commits.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, fields

import torch

INT64_MAX = torch.iinfo(torch.long).max


@dataclass
class MemoryState:
    keys: torch.Tensor            # [B, G, K_cap, D]
    values: torch.Tensor          # [B, G, K_cap, D]
    scores: torch.Tensor          # [B, G, K_cap] f32, -inf = empty
    positions: torch.Tensor       # [B, G, K_cap] i32, -1 = empty (the validity mask)
    pending_keys: torch.Tensor    # [B, G, PC, D]
    pending_values: torch.Tensor  # [B, G, PC, D]
    pending_scores: torch.Tensor  # [B, G, PC] f32
    count: torch.Tensor           # [B] i64
    total: torch.Tensor           # [B] i64

    @classmethod
    def empty(cls, batch, groups, capacity, chunk, dim, dtype=torch.bfloat16):
        kv = (batch, groups, capacity, dim)
        pend = (batch, groups, chunk, dim)
        return cls(torch.zeros(kv, dtype=dtype), torch.zeros(kv, dtype=dtype),
                   torch.full(kv[:-1], -math.inf), torch.full(kv[:-1], -1, dtype=torch.int32),
                   torch.zeros(pend, dtype=dtype), torch.zeros(pend, dtype=dtype),
                   torch.full(pend[:-1], -math.inf), torch.zeros(batch, dtype=torch.long),
                   torch.zeros(batch, dtype=torch.long))

    def clone(self) -> "MemoryState":
        return MemoryState(*(getattr(self, f.name).clone() for f in fields(self)))

    def to(self, device) -> "MemoryState":
        return MemoryState(*(getattr(self, f.name).to(device) for f in fields(self)))


def select_topk(scores, positions, references, capacity):
    """Keep the best ``capacity`` candidates along the last dim
    (modeling_yanchor.py:51-60).  Returns (scores, positions, references),
    padded with (-inf, -1, -1) when there are fewer candidates."""
    positions = positions.long().masked_fill(references < 0, -1)
    pos_key = positions.masked_fill(references < 0, INT64_MAX)
    order = pos_key.argsort(dim=-1, stable=True)
    scores, positions, references = (x.gather(-1, order) for x in (scores, positions, references))
    order = scores.argsort(dim=-1, descending=True, stable=True)[..., :capacity]
    out = [x.gather(-1, order) for x in (scores, positions, references)]
    missing = capacity - order.shape[-1]
    if missing:
        out = [torch.nn.functional.pad(x, (0, missing), value=v)
               for x, v in zip(out, (-math.inf, -1, -1))]
    return tuple(out)


def merge_topk(left, right, capacity):
    """Top-K of the concatenation of two candidate lists (modeling_yanchor.py:62-63)."""
    return select_topk(*(torch.cat((a, b), -1) for a, b in zip(left, right)), capacity)


def select_topk_bruteforce(scores, positions, references, capacity):
    """The same selection with Python's sorted() on one 1-D candidate list."""
    items = []
    for i, (s, p, r) in enumerate(zip(scores.tolist(), positions.tolist(), references.tolist())):
        p = -1 if r < 0 else int(p)
        pk = INT64_MAX if r < 0 else p
        items.append((-(s + 0.0), pk, i, s, p, r))  # s + 0.0 maps -0.0 to +0.0
    items.sort(key=lambda x: (x[0], x[1], x[2]))
    chosen = items[:capacity]
    out_s = [c[3] for c in chosen] + [-math.inf] * (capacity - len(chosen))
    out_p = [c[4] for c in chosen] + [-1] * (capacity - len(chosen))
    out_r = [c[5] for c in chosen] + [-1] * (capacity - len(chosen))
    return out_s, out_p, out_r


def exclusive_prefix_topk(scores, positions, references, capacity):
    """For every block j of ``[B, NB, G, C]`` candidates: Top-K over all
    candidates in blocks < j (an empty set for j = 0), plus a final entry
    j = NB over all blocks.  Returns tensors ``[B, NB + 1, G, capacity]``.
    Definition form of modeling_yanchor.py:65-78 (the reference computes it
    with an up-sweep / down-sweep tree of merge_topk)."""
    b, nb, g, c = scores.shape
    outs = ([], [], [])
    for j in range(nb + 1):
        s = scores[:, :j].permute(0, 2, 1, 3).reshape(b, g, j * c)
        p = positions[:, :j].permute(0, 2, 1, 3).reshape(b, g, j * c)
        r = references[:, :j].permute(0, 2, 1, 3).reshape(b, g, j * c)
        sel = select_topk(s, p, r, capacity)
        for o, x in zip(outs, sel):
            o.append(x)
    return tuple(torch.stack(o, 1) for o in outs)


def _rows(batch, indices):
    if indices is None:
        return list(range(batch))
    return [int(i) for i in indices.tolist()]


def indexed_gqa(query, key, value, references, dtype=torch.float64):
    """Prefill read of referenced source rows (modeling_yanchor.py:22-42;
    runtime/model/independent_memory.py:6-45).

    query ``[B, NB, C, H, D]``; key, value ``[KB, S, G, D]`` (KB == B, or 1 =
    one source for every row, as the Triton kernel's key_batch); references
    ``[B, NB, G, CAP]`` (-1 = none).  For row b, block nb, group g: the queries
    of heads g*R .. g*R+R-1 (R = H / G) at every block position attend over
    key/value rows ``references[b, nb, g, :]`` with logits q.k / sqrt(D) and
    one extra logit 0 whose value is 0 (the padded zero key / value row of
    _gqa_tile, the max-0 / denominator-1 start of _indexed_forward)."""
    b, nb, c, h, d = query.shape
    kb, s, g, _ = key.shape
    r = h // g
    out = torch.zeros(b, nb, c, h, d, dtype=dtype)
    for bi in range(b):
        src = 0 if kb == 1 else bi
        for blk in range(nb):
            for gi in range(g):
                refs = references[bi, blk, gi].long()
                ok = (refs >= 0) & (refs < s)
                idx = refs.clamp(0, max(s - 1, 0))
                keys = key[src, idx, gi].to(dtype)                            # [CAP, D]
                vals = value[src, idx, gi].to(dtype)
                q = query[bi, blk, :, gi * r:(gi + 1) * r].to(dtype)          # [C, R, D]
                logits = (q @ keys.T / math.sqrt(d)).masked_fill(~ok, -math.inf)
                w = torch.nn.functional.pad(logits, (0, 1), value=0.0).softmax(-1)[..., :-1]
                out[bi, blk, :, gi * r:(gi + 1) * r] = w @ vals
    return out.to(query.dtype)


def committed_read(query, state: MemoryState, indices=None, dtype=torch.float64):
    """Decode read of the committed slots (modeling_yanchor.py:283-290).

    query ``[B, 1, H, D]``; H = G * R with query head h reading group h // R.
    Per (row, head): logits = q.K^T / sqrt(D) over slots whose position >= 0;
    weights = softmax([logits, 0])[:-1] (a sink logit of 0 with value 0);
    read = weights @ V, cast to the query dtype.  With ``indices`` row r reads
    state row indices[r]; a negative index reads nothing (output 0)."""
    bq, _, h, d = query.shape
    g = state.keys.shape[1]
    r = h // g
    out = torch.zeros(bq, 1, h, d, dtype=dtype)
    for row, b in enumerate(_rows(bq, indices)):
        if b < 0:
            continue
        q = query[row, 0].to(dtype).reshape(g, r, d)
        keys = state.keys[b].to(dtype)
        vals = state.values[b].to(dtype)
        logits = q @ keys.transpose(-1, -2) / math.sqrt(d)               # [G, R, K]
        logits = logits.masked_fill((state.positions[b] < 0)[:, None, :], -math.inf)
        w = torch.nn.functional.pad(logits, (0, 1), value=0.0).softmax(-1)[..., :-1]
        out[row, 0] = (w @ vals).reshape(h, d)
    return out.to(query.dtype)


def commit_decode(key, value, scores, active, chunk, state: MemoryState, indices=None):
    """Push one token per row and commit a full chunk, IN PLACE on ``state``
    (modeling_yanchor.py:291-312; independent_memory.py:90-175).

    key, value ``[B, 1, G, D]``; scores ``[B, 1, G]`` fp32; active ``[B]`` bool.
    For each active row (state row b = indices[row] or row, skipped if < 0):
    write (key, value, score) to pending slot ``count[b]``; if that fills the
    chunk (count + 1 == chunk) replace the committed slots of every group by
    the Top-K_cap of committed + pending candidates (pending j has position
    total - count + j) and reset count to 0, else count += 1; total += 1."""
    bsz = key.shape[0]
    g_n, cap, d = state.keys.shape[1:]
    for row, b in enumerate(_rows(bsz, indices)):
        if b < 0 or not bool(active[row]):
            continue
        c = int(state.count[b])
        state.pending_keys[b, :, c] = key[row, 0]
        state.pending_values[b, :, c] = value[row, 0]
        state.pending_scores[b, :, c] = scores[row, 0]
        if c + 1 == chunk:
            base = int(state.total[b]) - c
            for g in range(g_n):
                pos = state.positions[b, g].long()
                ref = torch.arange(cap).masked_fill(pos < 0, -1)
                cand_s = torch.cat((state.scores[b, g], state.pending_scores[b, g, :chunk]))
                cand_p = torch.cat((pos, base + torch.arange(chunk)))
                cand_r = torch.cat((ref, cap + torch.arange(chunk)))
                ss, pp, rr = select_topk_bruteforce(cand_s, cand_p, cand_r, cap)
                src_k = torch.cat((state.keys[b, g], state.pending_keys[b, g, :chunk]))
                src_v = torch.cat((state.values[b, g], state.pending_values[b, g, :chunk]))
                take = torch.tensor([max(x, 0) for x in rr])
                state.keys[b, g] = src_k[take]
                state.values[b, g] = src_v[take]
                state.scores[b, g] = torch.tensor(ss, dtype=torch.float32)
                state.positions[b, g] = torch.tensor(pp, dtype=torch.int32)
            state.count[b] = 0
        else:
            state.count[b] = c + 1
        state.total[b] += 1
    return state


def committed_read_batched(query, state: MemoryState, dtype=torch.float32):
    """committed_read for every row at once (the torch branch of _decode,
    modeling_yanchor.py:283-290): one batched product per group, masked
    logits, the zero-logit sink, in ``dtype``."""
    bq, _, h, d = query.shape
    g = state.keys.shape[1]
    q = query[:, 0].to(dtype).reshape(bq, g, h // g, d)
    logits = q @ state.keys.to(dtype).transpose(-1, -2) / math.sqrt(d)           # [B, G, R, K]
    logits = logits.masked_fill((state.positions < 0)[:, :, None, :], -math.inf)
    w = torch.nn.functional.pad(logits, (0, 1), value=0.0).softmax(-1)[..., :-1]
    return (w @ state.values.to(dtype)).reshape(bq, 1, h, d).to(query.dtype)


def commit_decode_batched(key, value, scores, active, chunk, state: MemoryState):
    """commit_decode for every row at once, IN PLACE (the torch branch of
    _decode, modeling_yanchor.py:291-313): the push into pending slot
    ``count``, then one select_topk over committed + pending candidates of
    every row whose chunk fills."""
    bsz = key.shape[0]
    g_n, cap, d = state.keys.shape[1:]
    rows = torch.arange(bsz)[:, None]
    grp = torch.arange(g_n)[None]
    slot = state.count.long()[:, None]
    act = active.bool()
    for target, src in ((state.pending_keys, key[:, 0]), (state.pending_values, value[:, 0])):
        target[rows, grp, slot] = torch.where(act[:, None, None], src.to(target.dtype), target[rows, grp, slot])
    state.pending_scores[rows, grp, slot] = torch.where(act[:, None], scores[:, 0].to(state.pending_scores.dtype),
                                                        state.pending_scores[rows, grp, slot])
    nxt = state.count.long() + act.long()
    commit = nxt == chunk
    cr = commit.nonzero()[:, 0]
    if cr.numel():
        n = cr.numel()
        pos = state.positions[cr].long()
        ref = torch.arange(cap).expand(n, g_n, cap).masked_fill(pos < 0, -1)
        base = (state.total[cr] - state.count[cr]).long()      # position of pending entry 0
        pj = torch.arange(chunk)
        cand_s = torch.cat((state.scores[cr], state.pending_scores[cr][:, :, :chunk]), -1)
        cand_p = torch.cat((pos, (base[:, None, None] + pj).expand(n, g_n, chunk)), -1)
        cand_r = torch.cat((ref, (cap + pj).expand(n, g_n, chunk)), -1)
        ss, pp, rr = select_topk(cand_s, cand_p, cand_r, cap)
        take = rr.clamp_min(0)[..., None].expand(n, g_n, cap, d)
        for target, pend in ((state.keys, state.pending_keys), (state.values, state.pending_values)):
            src = torch.cat((target[cr], pend[cr][:, :, :chunk]), 2)
            target[cr] = src.gather(2, take)
        state.scores[cr] = ss.to(state.scores.dtype)
        state.positions[cr] = pp.to(state.positions.dtype)
    state.count.copy_(torch.where(commit, torch.zeros_like(nxt), nxt).to(state.count.dtype))
    state.total.add_(act.to(state.total.dtype))
    return state


def sequence(query, key, value, scores, valid, chunk, state: MemoryState, dtype=torch.float64):
    """Anchor-memory read and write of a prefill chunk continuing ``state``,
    IN PLACE (IndependentGQAMemory._sequence with a state,
    modeling_yanchor.py:178-275), restated step by step: order the valid
    tokens first (180-187); place them after the old pending tokens in an
    extended sequence of whole chunks (189-206); exclusive prefix Top-K of the
    blocks merged with the committed slots (207-219); every block's queries
    read the memory in force before it (244-250); the state keeps the memory
    after the last full block and the tokens after it as pending (256-274).

    query ``[B, L, H, D]``; key, value ``[B, L, G, D]`` (every token's written
    key / value: the reference writes only the tokens it will read, 220-231,
    which changes no result); scores ``[B, L, G]``; valid ``None`` or bool
    ``[B, L]``.  Returns ``[B, L, H, D]`` in the query dtype."""
    b, length, h, d = query.shape
    g_n, cap = state.keys.shape[1], state.keys.shape[2]
    c = int(chunk)
    bi = torch.arange(b)[:, None]
    if valid is None:
        order = None
        q, k, v, s = query, key, value, scores
        counts = torch.full((b,), length, dtype=torch.long)
    else:
        order = valid.long().argsort(dim=1, descending=True, stable=True)
        q, k, v, s = (x[bi, order] for x in (query, key, value, scores))
        counts = valid.long().sum(1)
    old_count, old_total = state.count.clone(), state.total.clone()
    extent = math.ceil((length + c) / c) * c
    at = torch.arange(extent)[None].expand(b, -1)
    valid_extent = at < (old_count + counts)[:, None]
    select = torch.where(at < old_count[:, None], at, c + at - old_count[:, None]).clamp_max(c + length - 1)
    qx = torch.cat((q.new_zeros(b, c, h, d), q), 1)[bi, select]
    sx = torch.cat((state.pending_scores.transpose(1, 2)[:, :c], s.float()), 1)[bi, select]
    sx = sx.masked_fill(~valid_extent[..., None], -math.inf)
    positions = (old_total - old_count)[:, None] + at
    refs = (at + cap).masked_fill(~valid_extent, -1)               # sequence index + committed slots
    blocks = extent // c
    meta = [x[:, :, None].expand(-1, -1, g_n) if x.ndim == 2 else x for x in (sx, positions, refs)]
    meta = [x.reshape(b, blocks, c, g_n).transpose(2, 3) for x in meta]
    prefix = exclusive_prefix_topk(*meta, cap)                      # [B, blocks + 1, G, cap]
    slots = torch.arange(cap)[None, None].expand(b, g_n, -1).masked_fill(state.positions < 0, -1)
    initial = (state.scores, state.positions, slots)
    prefix = merge_topk(prefix, tuple(x[:, None].expand(-1, blocks + 1, -1, -1) for x in initial), cap)
    # source rows: committed slot s -> s; old pending t -> cap + t; new token i -> cap + c + i
    src_k = torch.cat((state.keys.transpose(1, 2), state.pending_keys[:, :, :c].transpose(1, 2), k), 1)
    src_v = torch.cat((state.values.transpose(1, 2), state.pending_values[:, :, :c].transpose(1, 2), v), 1)
    table = torch.full((b, cap + extent), -1, dtype=torch.long)    # reference -> source row
    table[:, :cap] = torch.arange(cap)
    t_idx = at
    table[:, cap:] = torch.where(t_idx < old_count[:, None], cap + t_idx,
                                 torch.where(valid_extent, cap + c + (t_idx - old_count[:, None]),
                                             torch.full_like(t_idx, -1)))
    def rows(r):
        return table[bi.reshape(b, *([1] * (r.ndim - 1))).expand_as(r), r.clamp_min(0)].masked_fill(r < 0, -1)
    read_refs = rows(prefix[2][:, :-1])                             # [B, blocks, G, cap]
    read = indexed_gqa(qx.reshape(b, blocks, c, h, d), src_k, src_v, read_refs, dtype=dtype).flatten(1, 2)
    out = read[bi, (old_count[:, None] + torch.arange(length)[None]).clamp_max(extent - 1)]
    if order is not None:
        out = out[bi, order.argsort(1)] * valid[..., None, None].to(out.dtype)
    full = (old_count + counts) // c
    score, position, reference = (x[torch.arange(b), full] for x in prefix)
    src_rows = rows(reference)                                      # [B, G, cap]
    g_idx = torch.arange(g_n)[None, :, None]
    b_idx = torch.arange(b)[:, None, None]
    state.keys.copy_(src_k[b_idx, src_rows.clamp_min(0), g_idx].masked_fill((src_rows < 0)[..., None], 0))
    state.values.copy_(src_v[b_idx, src_rows.clamp_min(0), g_idx].masked_fill((src_rows < 0)[..., None], 0))
    state.scores.copy_(score)
    state.positions.copy_(position.to(torch.int32))
    pc = state.pending_keys.shape[2]
    remaining = (old_count + counts) % c
    pend = (full[:, None] * c + torch.arange(pc)[None]).clamp_max(extent - 1)   # sequence indices
    mask = torch.arange(pc)[None] < remaining[:, None]
    prow = table[bi, cap + pend].clamp_min(0)                       # [B, pc]
    state.pending_keys.copy_(src_k[bi, prow].masked_fill(~mask[..., None, None], 0).transpose(1, 2))
    state.pending_values.copy_(src_v[bi, prow].masked_fill(~mask[..., None, None], 0).transpose(1, 2))
    state.pending_scores.copy_(sx[bi, pend].masked_fill(~mask[..., None], -math.inf).transpose(1, 2))
    state.count.copy_(remaining)
    state.total.add_(counts)
    return out
