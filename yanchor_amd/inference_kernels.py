"""Sampling and slot-management kernels behind the reference's call signatures.

Mirrors the names of runtime/model/inference_kernels.py:

* ``counter_uniform``                  24-33
* ``sample_top_k_top_p_counter``       73-88  (torch-sampler semantics)
* ``_sample_top_k_top_p_counter_triton`` 1147-1167 (fused top-20 semantics);
  also exported as ``sample_top20_counter``
* ``_apply_dense_presence_penalty_``   1104-1114
* ``_update_fixed_decode_state_``      1206-1208
* refill targets / compaction keep-list (``torch.nonzero`` at 1549 and 1725),
  ``cu_seqlens`` for packed prefill and the cache row gather/scatter.

Every function runs a HIP kernel from the yanchor_amd library on the tensors'
device and raises for CPU tensors.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as N

COUNTER_SAMPLING_REVISION = "counter_cdf_v2"
SAMPLE_FUSED, SAMPLE_TORCH = 0, 1
SELECT_KEEP, SELECT_FINISHED = 0, 1

_workspaces: dict[tuple, torch.Tensor] = {}


def topk_workspace(batch: int, vocab: int, top_k: int, device) -> torch.Tensor:
    """Cached device workspace for the sampler (allocated once per shape, so a
    graph-captured decode step does not allocate)."""
    key = (torch.device(device), int(batch), int(vocab), int(top_k))
    ws = _workspaces.get(key)
    if ws is None:
        nbytes = int(N.lib().yh_topk_workspace_bytes(batch, vocab, top_k))
        ws = torch.empty(max(8, nbytes), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _steps_arg(steps, batch, device):
    if isinstance(steps, torch.Tensor):
        if steps.shape != (batch,) or steps.dtype not in (torch.int32, torch.int64):
            raise ValueError("steps must be one integer per row")
        return steps.to(device=device, dtype=torch.int64).contiguous(), 0
    return None, int(steps)


def counter_uniform(attempt_ids, steps, *, seed: int, stream: int = 0, dtype=torch.float32):
    """Uniform draws in (0, 1) from the counter hash (inference_kernels.py:24-33)."""
    if attempt_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("attempt ids must be integer tensors")
    if dtype != torch.float32:
        raise ValueError("counter_uniform on the GPU produces float32")
    N.require_device(attempt_ids)
    ids = attempt_ids.to(torch.int64).contiguous()
    st, step = _steps_arg(steps, ids.shape[0], ids.device)
    out = torch.empty(ids.shape, dtype=torch.float32, device=ids.device)
    N.call("yh_counter_uniform", ids.data_ptr(), N.ptr(st), step, int(seed) & 0xFFFFFFFF,
           int(stream) & 0xFFFFFFFF, out.data_ptr(), ids.numel(), N.stream_of(ids))
    return out


def topk_sample(scores, attempt_ids, steps, *, seed, temperature, top_k, top_p, mode, stream=0,
                seen=None, presence_penalty=0.0, return_topk=False):
    """One token per row ([B, 1] int64) from the top-k of ``scores`` [B, V]
    (fp32 / bf16 / fp16; rows may be a strided view such as
    ``logits[:, :vocab]``), with the dense presence penalty of ``seen`` fused
    in (scores are not modified)."""
    if scores.ndim != 2 or scores.stride(1) != 1:
        raise ValueError("sampling scores must have shape [batch, vocabulary] with unit column stride")
    b, v = scores.shape
    top_k = int(top_k)
    full = top_k <= 0 or top_k > 64
    if full and (mode != SAMPLE_TORCH or return_topk):
        raise ValueError("top_k outside [1, 64] is the torch sampler's full-vocabulary branch (no top-k output)")
    if top_k > v:   # every branch, as the reference refuses it (inference_kernels.py:46-47)
        raise ValueError("top-k exceeds the vocabulary")
    if top_k != 1 and (temperature <= 0.0 or not 0.0 < top_p <= 1.0):
        raise ValueError("invalid top-k/top-p sampling parameters")
    if attempt_ids.shape != (b,):
        raise ValueError("attempt ids must contain one id per row")
    dev = N.require_device(scores, attempt_ids, seen)
    ids = attempt_ids.to(torch.int64).contiguous()
    st, step = _steps_arg(steps, b, dev)
    seen_ptr, seen_stride = None, 0
    if seen is not None and presence_penalty != 0.0:
        if seen.shape != scores.shape or seen.dtype != torch.bool or seen.stride(1) != 1:
            raise ValueError("dense presence state must be a boolean scores-shaped tensor")
        seen_ptr, seen_stride = seen.data_ptr(), seen.stride(0)
    ws = None if full else topk_workspace(b, v, top_k, dev)
    tokens = torch.empty(b, 1, dtype=torch.int64, device=dev)
    vals = idxs = None
    if return_topk:
        vals = torch.empty(b, top_k, dtype=torch.float32, device=dev)
        idxs = torch.empty(b, top_k, dtype=torch.int64, device=dev)
    N.call("yh_topk_sample", scores.data_ptr(), N.code(scores), scores.stride(0), seen_ptr, seen_stride,
           float(presence_penalty), ids.data_ptr(), N.ptr(st), step, int(seed) & 0xFFFFFFFF,
           int(stream) & 0xFFFFFFFF, float(temperature) if top_k != 1 else 1.0, int(top_k),
           float(top_p) if top_k != 1 else 1.0, int(mode), tokens.data_ptr(), N.ptr(vals), N.ptr(idxs),
           N.ptr(ws), 0 if ws is None else ws.numel(), b, v, N.stream_of(scores))
    return (tokens, vals, idxs) if return_topk else tokens


def sample_top_k_top_p_counter(scores, attempt_ids, steps, *, seed, temperature, top_k, top_p, stream=0):
    """Torch-sampler semantics (inference_kernels.py:73-88), every branch:
    top_k <= 0 with top_p == 1 draws over the whole vocabulary in vocabulary
    order; top_k == 1 is the argmax; otherwise the top k (the whole
    vocabulary for top_k <= 0) truncated at top_p.  top_k > V is refused as
    the reference refuses it (42-48)."""
    if int(top_k) > scores.shape[-1]:
        raise ValueError("top-k exceeds the vocabulary")
    return topk_sample(scores, attempt_ids, steps, seed=seed, temperature=temperature, top_k=top_k,
                       top_p=top_p, mode=SAMPLE_TORCH, stream=stream)


def sample_top20_counter(scores, attempt_ids, step, *, seed, temperature, top_k=20, top_p=0.95,
                         seen=None, presence_penalty=0.0):
    """Fused top-k sampler semantics (_qwen35_top20_counter_sample_kernel,
    inference_kernels.py:1119-1167), optionally with the presence penalty fused."""
    return topk_sample(scores, attempt_ids, step, seed=seed, temperature=temperature, top_k=top_k,
                       top_p=top_p, mode=SAMPLE_FUSED, seen=seen, presence_penalty=presence_penalty)


def _sample_top_k_top_p_counter_triton(scores, attempt_ids, step, *, seed, temperature, top_k, top_p):
    if top_k != 20 or not 0.0 < top_p <= 1.0 or temperature <= 0.0:
        raise ValueError("fused counter sampler requires top20 scores")
    return sample_top20_counter(scores, attempt_ids, step, seed=seed, temperature=temperature, top_k=top_k,
                                top_p=top_p)


def _apply_dense_presence_penalty_(scores, seen, penalty):
    """scores -= penalty where seen, in place (inference_kernels.py:1104-1114)."""
    if penalty == 0.0:
        return
    if scores.shape != seen.shape or seen.dtype != torch.bool:
        raise ValueError("dense presence state must be a boolean scores-shaped tensor")
    if scores.dtype != torch.float32 or not scores.is_contiguous() or not seen.is_contiguous():
        raise ValueError("presence penalty needs contiguous float32 scores")
    N.require_device(scores, seen)
    N.call("yh_presence_penalty", scores.data_ptr(), seen.data_ptr(), scores.numel(), float(penalty),
           N.stream_of(scores))


def _update_fixed_decode_state_(sampled_token, storage, dense_seen, generated_lengths, finished_by_eos,
                                finished, slot_rows, sink_rows, slot_caps, row_steps, row_positions,
                                decode_ids, decode_useful_events, *, maximum_new_tokens, pad_token_id,
                                eos_token_ids):
    """Per-step slot bookkeeping, in place (inference_kernels.py:1169-1208)."""
    slots = sampled_token.shape[0]
    checks = [(sampled_token, torch.int64), (storage, torch.int32), (dense_seen, torch.bool),
              (generated_lengths, torch.int64), (finished_by_eos, torch.bool), (finished, torch.bool),
              (slot_rows, torch.int64), (sink_rows, torch.int64), (slot_caps, torch.int64),
              (row_steps, torch.int64), (row_positions, torch.int64), (decode_ids, torch.int64),
              (decode_useful_events, torch.int64)]
    for t, dt in checks:
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"bookkeeping tensor of dtype {t.dtype} must be contiguous {dt}")
    if row_positions.ndim != 1:
        raise ValueError("bookkeeping needs [slots] row positions")
    N.require_device(sampled_token, storage, dense_seen, generated_lengths, finished_by_eos, finished)
    eos = (ctypes.c_int64 * max(1, len(eos_token_ids)))(*[int(x) for x in eos_token_ids])
    N.call("yh_decode_bookkeeping", sampled_token.data_ptr(), storage.data_ptr(), dense_seen.data_ptr(),
           generated_lengths.data_ptr(), finished_by_eos.data_ptr(), finished.data_ptr(), slot_rows.data_ptr(),
           sink_rows.data_ptr(), slot_caps.data_ptr(), row_steps.data_ptr(), row_positions.data_ptr(),
           decode_ids.data_ptr(), decode_useful_events.data_ptr(), slots, storage.shape[0], storage.shape[1],
           dense_seen.shape[1], int(maximum_new_tokens), int(pad_token_id),
           ctypes.cast(eos, ctypes.c_void_p).value, len(eos_token_ids), N.stream_of(storage))


def _initial_attempt_order(difficulty, attempt_ids, prefill_group_ids=None):
    """Order in which attempts take the physical slots at the start
    (inference_kernels.py:1321-1329): hardest first (largest ``difficulty``,
    the per-attempt generation cap), ties by ascending attempt id.  With
    prefill groups, whole groups move together: groups ordered by their
    hardest member, then their smallest attempt id; members inside a group in
    the same row order.  Returns row indices into ``attempt_ids``."""
    diff = [float(x) for x in (difficulty.tolist() if torch.is_tensor(difficulty) else difficulty)]
    ids = [int(x) for x in attempt_ids]

    def row_key(r):
        return -diff[r], ids[r]

    if prefill_group_ids is None:
        return sorted(range(len(ids)), key=row_key)
    members: dict[int, list[int]] = {}
    for r, gid in enumerate(prefill_group_ids):
        members.setdefault(int(gid), []).append(r)
    groups = sorted(members.values(), key=lambda rows: (-max(diff[r] for r in rows), min(ids[r] for r in rows)))
    return [r for rows in groups for r in sorted(rows, key=row_key)]


def _group_aligned_prefix_length(ordered_rows, prefill_group_ids, limit):
    """The longest prefix of ``ordered_rows`` with at most ``limit`` rows
    that ends on a prefill-group boundary (inference_kernels.py:1331-1346);
    a first group larger than ``limit`` is refused."""
    if limit <= 0 or not ordered_rows:
        return 0
    accepted = 0
    while accepted < len(ordered_rows):
        gid = int(prefill_group_ids[ordered_rows[accepted]])
        stop = accepted + 1
        while stop < len(ordered_rows) and int(prefill_group_ids[ordered_rows[stop]]) == gid:
            stop += 1
        if stop > limit:
            break
        accepted = stop
    if accepted == 0:
        raise ValueError(f"prefill group {int(prefill_group_ids[ordered_rows[0]])} is larger than the "
                         "ready-bank limit")
    return accepted


def _should_compact_dynamic_decode_tail(live_slots, physical_slots, *, queue_exhausted, live_fraction):
    """Tail-compaction trigger (inference_kernels.py:1348-1349): no more work
    queued and at most ``live_fraction`` of the physical slots live."""
    return bool(queue_exhausted and 0 < live_slots < physical_slots
                and live_slots <= max(1, int(physical_slots * live_fraction)))


def select_slots(finished, slot_rows=None, *, mode):
    """(indices [n] int64 with -1 padding, count [1] int64) of the rows that
    satisfy the mode, ascending; stays on the device."""
    if finished.dtype != torch.bool or finished.ndim != 1:
        raise ValueError("finished must be a boolean vector")
    n = finished.shape[0]
    dev = N.require_device(finished, slot_rows)
    rows = None
    if slot_rows is not None:
        if slot_rows.shape != (n,):
            raise ValueError("slot_rows must match finished")
        rows = slot_rows.to(torch.int64).contiguous()
    fin = finished.contiguous()
    out = torch.empty(n, dtype=torch.int64, device=dev)
    count = torch.empty(1, dtype=torch.int64, device=dev)
    N.call("yh_select_slots", fin.data_ptr(), N.ptr(rows), int(mode), out.data_ptr(), count.data_ptr(), n,
           N.stream_of(fin))
    return out, count


def compaction_keep(finished, slot_rows):
    """Ascending slots that are live (not finished, mapped to a row): the
    tail-compaction keep-list (inference_kernels.py:1725).  Syncs for the count."""
    out, count = select_slots(finished, slot_rows, mode=SELECT_KEEP)
    return out[: int(count.item())]


def refill_targets(finished):
    """Ascending finished slots: the refill targets (inference_kernels.py:1549).
    Syncs for the count."""
    out, count = select_slots(finished, None, mode=SELECT_FINISHED)
    return out[: int(count.item())]


def cu_seqlens(lengths):
    """int32 [N + 1] exclusive prefix sum of sequence lengths."""
    if lengths.ndim != 1 or lengths.dtype not in (torch.int32, torch.int64):
        raise ValueError("lengths must be a 1-D integer tensor")
    N.require_device(lengths)
    src = lengths.contiguous()
    out = torch.empty(src.shape[0] + 1, dtype=torch.int32, device=src.device)
    N.call("yh_cu_seqlens", src.data_ptr(), N.code(src), out.data_ptr(), src.shape[0], N.stream_of(src))
    return out


def gather_rows(pairs, src_index=None, dst_index=None, n=None):
    """For every (src, dst) pair of tensors: dst[dst_index[i]] = src[src_index[i]]
    along dim 0 (None = identity), in one launch per 32 tensors.  src and dst
    must be different tensors with equal per-row layout."""
    if not pairs:
        return
    if n is None:
        n = (src_index if src_index is not None else dst_index).shape[0]
    devs = [t for pair in pairs for t in pair] + [src_index, dst_index]
    N.require_device(*devs)
    cnt = len(pairs)
    srcp = (ctypes.c_void_p * cnt)()
    dstp = (ctypes.c_void_p * cnt)()
    rb = (ctypes.c_int64 * cnt)()
    sr = (ctypes.c_int64 * cnt)()
    dr = (ctypes.c_int64 * cnt)()
    for i, (s, d) in enumerate(pairs):
        if s.dtype != d.dtype or s.shape[1:] != d.shape[1:]:
            raise ValueError("gather_rows pairs must share dtype and row shape")
        if not s.is_contiguous() or not d.is_contiguous():
            raise ValueError("gather_rows needs contiguous tensors")
        srcp[i], dstp[i] = s.data_ptr(), d.data_ptr()
        rb[i] = s[0].numel() * s.element_size() if s.shape[0] else d[0].numel() * d.element_size()
        sr[i], dr[i] = s.shape[0], d.shape[0]
    si = None if src_index is None else src_index.to(torch.int64).contiguous()
    di = None if dst_index is None else dst_index.to(torch.int64).contiguous()
    N.call("yh_gather_rows", cnt, ctypes.cast(srcp, ctypes.c_void_p).value,
           ctypes.cast(dstp, ctypes.c_void_p).value, ctypes.cast(rb, ctypes.c_void_p).value,
           ctypes.cast(sr, ctypes.c_void_p).value, ctypes.cast(dr, ctypes.c_void_p).value, N.ptr(si),
           N.ptr(di), int(n), N.stream_of(pairs[0][0]))
