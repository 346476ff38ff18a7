"""Continuous-batch slot management on the CPU (oracle; test infrastructure only).

Restates runtime/model/inference_kernels.py:

* ``decode_state_update``       the fused bookkeeping kernel 1169-1204
* ``decode_state_update_torch`` the reference's torch fallback of the same step
                                1700-1718 (a second formulation; the tests check
                                the two agree)
* ``refill_targets``            nonzero(finished), ascending (1549)
* ``compaction_keep``           nonzero(~finished & slot_rows >= 0) (1725)
* ``should_compact``            _should_compact_dynamic_decode_tail (1348-1349)
* ``cu_seqlens``                exclusive prefix sum of packed lengths
* ``initial_attempt_order``     _initial_attempt_order (1321-1329)
* ``group_aligned_prefix``      _group_aligned_prefix_length (1331-1346)
* ``prefill_expansion``         build_prefill_expansion (90-121): representative
                                row of each prefill group and every row's group

Integer work, bit-exact; Python ints and torch integer tensors on the CPU.
"""
from __future__ import annotations

import torch


def decode_state_update(sampled, storage, dense_seen, generated_lengths, finished_by_eos, finished,
                        slot_rows, sink_rows, slot_caps, row_steps, row_positions, decode_ids, useful, *,
                        maximum_new_tokens, pad_token_id, eos_token_ids):
    """Row loop of _qwen35_decode_state_update_kernel (1169-1204), in place."""
    eos = list(eos_token_ids)[:2]
    count = 0
    for r in range(sampled.shape[0]):
        tok = int(sampled.reshape(-1)[r])
        fin = bool(finished[r])
        row = int(slot_rows[r])
        active = (not fin) and row >= 0
        step = int(row_steps[r])
        wrow = row if active else int(sink_rows[r])
        wcol = step if active else int(maximum_new_tokens)
        stored = tok if active else int(pad_token_id)
        storage[wrow, wcol] = stored
        dense_seen[r, stored] = True
        nstep = step + int(active)
        if active:
            generated_lengths[wrow] = nstep
        is_eos = stored in eos
        if active and is_eos:
            finished_by_eos[wrow] = True
        nfin = fin or (active and (is_eos or nstep >= int(slot_caps[r])))
        finished[r] = nfin
        row_steps[r] = nstep
        row_positions[r] += int(active)
        decode_ids.reshape(-1)[r] = pad_token_id if nfin else stored
        count += int(active)
    useful += count


def decode_state_update_torch(sampled, storage, dense_seen, generated_lengths, finished_by_eos, finished,
                              slot_rows, sink_rows, slot_caps, row_steps, row_positions, decode_ids, useful, *,
                              maximum_new_tokens, pad_token_id, eos_token_ids):
    """The reference's vectorised fallback of the same step (1700-1718)."""
    active = ~finished & (slot_rows >= 0)
    tok = torch.where(active[:, None], sampled, sampled.new_full((), pad_token_id))
    wrows = torch.where(active, slot_rows, sink_rows)
    wcols = torch.where(active, row_steps, row_steps.new_full((), maximum_new_tokens))
    storage[wrows, wcols] = tok[:, 0].to(storage.dtype)
    dense_seen.scatter_(1, tok, True)
    nsteps = row_steps + active.to(row_steps.dtype)
    generated_lengths[wrows] = torch.where(active, nsteps, generated_lengths[wrows])
    is_eos = torch.zeros_like(finished)
    for t in eos_token_ids:
        is_eos |= tok[:, 0] == int(t)
    finished_by_eos[wrows] |= active & is_eos
    finished |= active & (is_eos | (nsteps >= slot_caps))
    row_steps.copy_(nsteps)
    row_positions.add_(active.to(row_positions.dtype))
    decode_ids.copy_(torch.where(finished[:, None], tok.new_full((), pad_token_id), tok))
    useful.add_(active.sum())


def refill_targets(finished):
    return [i for i, f in enumerate(finished.tolist()) if f]


def compaction_keep(finished, slot_rows):
    return [i for i, (f, r) in enumerate(zip(finished.tolist(), slot_rows.tolist())) if (not f) and r >= 0]


def should_compact(live_slots, physical_slots, *, queue_exhausted, live_fraction):
    return (queue_exhausted and 0 < live_slots < physical_slots
            and live_slots <= max(1, int(physical_slots * live_fraction)))


def cu_seqlens(lengths):
    out = [0]
    for n in lengths:
        out.append(out[-1] + int(n))
    return out


def initial_attempt_order(difficulty, attempt_ids, groups=None):
    """Rows ordered hardest first (largest difficulty, then smallest attempt
    id); with prefill groups, whole groups: by their hardest member, then
    their smallest attempt id, rows inside a group by the same key.  Pinned
    by hand-worked orders (tests/test_host_logic.py)."""
    key = {r: (-float(difficulty[r]), int(attempt_ids[r])) for r in range(len(attempt_ids))}
    if groups is None:
        return sorted(key, key=key.get)
    members = {}
    for r, gid in enumerate(groups):
        members.setdefault(int(gid), []).append(r)
    ordered = sorted(members.values(), key=lambda rows: (min(key[r][0] for r in rows), min(key[r][1] for r in rows)))
    return [r for rows in ordered for r in sorted(rows, key=key.get)]


def group_aligned_prefix(ordered_rows, groups, limit):
    """The longest prefix of at most ``limit`` rows that ends where a group
    ends; ValueError when the first group alone exceeds ``limit``."""
    if limit <= 0 or not ordered_rows:
        return 0
    ends = [i + 1 for i in range(len(ordered_rows))
            if i + 1 == len(ordered_rows) or groups[ordered_rows[i + 1]] != groups[ordered_rows[i]]]
    fit = [e for e in ends if e <= limit]
    if not fit:
        raise ValueError("the first prefill group is larger than the limit")
    return fit[-1]


def prefill_expansion(groups):
    """(representative rows, inverse): the first row of each group in row
    order, and for every row the index of its group's representative."""
    first, inverse = {}, []
    for r, gid in enumerate(groups):
        first.setdefault(int(gid), len(first))
        inverse.append(first[int(gid)])
    reps = [0] * len(first)
    for r, gid in reversed(list(enumerate(groups))):
        reps[first[int(gid)]] = r
    return reps, inverse
