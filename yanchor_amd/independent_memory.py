"""Anchor-memory kernels behind the reference's ``model.independent_memory`` API.

The reference imports this module through ``_cuda_module('independent_memory')``
(modeling_yanchor.py:19-20, used at 249 and 278-282) and calls
``indexed_gqa(query, key, value, references)`` (prefill),
``committed_gqa(query, state, indices)`` and
``commit_decode(key, value, scores, active, chunk, state, indices)``
(runtime/model/independent_memory.py:177-201).  ``sequence`` is the stateful
prefill continuation of IndependentGQAMemory._sequence
(modeling_yanchor.py:178-275) on the GPU.  ``IndependentMemoryState``
mirrors the reference dataclass (modeling_yanchor.py:80-120) field for field, so
a state built by either side works with the other.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, fields

import torch

from . import _native as N


@dataclass
class IndependentMemoryState:
    keys: torch.Tensor            # [B, G, K_cap, D]
    values: torch.Tensor          # [B, G, K_cap, D]
    scores: torch.Tensor          # [B, G, K_cap] float32, -inf = empty
    positions: torch.Tensor       # [B, G, K_cap] int32, -1 = empty
    pending_keys: torch.Tensor    # [B, G, C_max, D]
    pending_values: torch.Tensor  # [B, G, C_max, D]
    pending_scores: torch.Tensor  # [B, G, C_max] float32
    count: torch.Tensor           # [B] int64
    total: torch.Tensor           # [B] int64

    @classmethod
    def empty(cls, batch, groups, capacity, chunk, dim, device, dtype):
        kv = (batch, groups, capacity, dim)
        pend = (batch, groups, chunk, dim)
        return cls(torch.zeros(kv, device=device, dtype=dtype), torch.zeros(kv, device=device, dtype=dtype),
                   torch.full(kv[:-1], -math.inf, device=device, dtype=torch.float32),
                   torch.full(kv[:-1], -1, device=device, dtype=torch.int32),
                   torch.zeros(pend, device=device, dtype=dtype), torch.zeros(pend, device=device, dtype=dtype),
                   torch.full(pend[:-1], -math.inf, device=device, dtype=torch.float32),
                   torch.zeros(batch, device=device, dtype=torch.long),
                   torch.zeros(batch, device=device, dtype=torch.long))

    def select(self, indices):
        return type(self)(*(getattr(self, f.name).index_select(0, indices.to(self.keys.device))
                            for f in fields(self)))

    def repeat(self, repeats):
        return type(self)(*(getattr(self, f.name).repeat_interleave(repeats, 0) for f in fields(self)))

    def scatter_(self, source, target_indices, source_indices):
        for f in fields(self):
            target, value = getattr(self, f.name), getattr(source, f.name)
            target.index_copy_(0, target_indices.to(target.device),
                               value.index_select(0, source_indices.to(value.device)).to(target.device))

    def reset_(self, rows=None):
        for f in fields(self):
            value = getattr(self, f.name)
            fill = -math.inf if "scores" in f.name else -1 if f.name == "positions" else 0
            if rows is None:
                value.fill_(fill)
            else:
                value.index_fill_(0, rows.to(value.device), fill)

    def to_(self, device):
        for f in fields(self):
            setattr(self, f.name, getattr(self, f.name).to(device, non_blocking=True))


def _check_state(state: IndependentMemoryState):
    b, g, cap, d = state.keys.shape
    if state.values.shape != state.keys.shape or state.values.dtype != state.keys.dtype:
        raise ValueError("memory keys and values must match")
    if state.scores.shape != (b, g, cap) or state.scores.dtype != torch.float32:
        raise ValueError("memory scores must be float32 [B, G, K_cap]")
    if state.positions.shape != (b, g, cap) or state.positions.dtype != torch.int32:
        raise ValueError("memory positions must be int32 [B, G, K_cap]")
    pc = state.pending_keys.shape[2]
    if state.pending_keys.shape != (b, g, pc, d) or state.pending_values.shape != (b, g, pc, d):
        raise ValueError("pending keys/values must be [B, G, C, D]")
    if state.pending_scores.shape != (b, g, pc) or state.pending_scores.dtype != torch.float32:
        raise ValueError("pending scores must be float32 [B, G, C]")
    if state.count.dtype != torch.long or state.total.dtype != torch.long:
        raise ValueError("count/total must be int64")
    if state.count.shape != (b,) or state.total.shape != (b,):
        raise ValueError("count/total must be [B]")
    return b, g, cap, pc, d


def _row_strides(state: IndependentMemoryState):
    """Elements between consecutive state rows of every field (field order).
    Each row must be dense inside; rows may sit in larger slot pages (the vLLM
    wire format keeps all fields of a slot in two page rows)."""
    out = []
    for f in fields(state):
        t = getattr(state, f.name)
        inner = t[0] if t.shape[0] else t
        if t.shape[0] and not inner.is_contiguous():
            raise ValueError(f"memory state field {f.name} must be dense within a row")
        out.append(t.stride(0) if t.shape[0] > 1 else math.prod(t.shape[1:]))
    return out


def _indices(indices, batch):
    if indices is None:
        return None
    if indices.shape != (batch,):
        raise ValueError("state indices must have one entry per batch row")
    return indices.to(torch.int32).contiguous()


def indexed_gqa(query, key, value, references):
    """Prefill read of the anchor memory (runtime/model/independent_memory.py:
    38-45; torch form modeling_yanchor.py:22-42).

    query ``[B, NB, C, H, D]``; key, value ``[KB, S, G, D]`` (KB == B, or 1 for
    a source shared by every row); references ``[B, NB, G, CAP]`` int32/int64
    rows of S (-1 = none).  Each query of block ``nb`` and head ``h`` attends
    over the referenced rows of group ``h // (H // G)`` with the zero-logit
    sink; returns ``[B, NB, C, H, D]`` in the query dtype."""
    if query.ndim != 5 or key.ndim != 4 or references.ndim != 4:
        raise ValueError("indexed_gqa expects query [B, NB, C, H, D], key/value [KB, S, G, D], "
                         "references [B, NB, G, CAP]")
    b, nb, c, h, d = query.shape
    kb, s, g, kd = key.shape
    if value.shape != key.shape or kd != d:
        raise ValueError("key/value must be [KB, S, G, D] with the query head dim")
    if references.shape[:3] != (b, nb, g):
        raise ValueError("references must be [B, NB, G, CAP]")
    if kb not in (1, b):
        raise ValueError("key batch must be 1 or B")
    if h % g:
        raise ValueError("query heads must be a multiple of the groups")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError("query, key and value must share a dtype")
    if references.dtype not in (torch.int32, torch.int64):
        raise ValueError("references must be int32 or int64")
    N.require_device(query, key, value, references)
    q, k, v, refs = (x.contiguous() for x in (query, key, value, references))
    out = torch.empty_like(q)
    N.call("yh_indexed_gqa", q.data_ptr(), k.data_ptr(), v.data_ptr(), refs.data_ptr(),
           N.DTYPE_CODE[refs.dtype], out.data_ptr(), b, nb, c, h, g, d, kb, s, refs.shape[-1], N.code(q),
           N.stream_of(q))
    return out


def committed_gqa(query, state: IndependentMemoryState, indices=None):
    """Read the committed anchor slots for one decode token.

    query ``[B, 1, H, D]``; returns ``[B, 1, H, D]`` in the query dtype: per
    head, softmax over [q.K^T / sqrt(D) on live slots, 0] applied to V (the
    zero-logit sink).  Row b reads state row ``indices[b]`` when given (-1 reads
    nothing and returns 0)."""
    return committed_gqa_gated(query, state, indices)


def committed_gqa_gated(query, state: IndependentMemoryState, indices=None, valid=None, head_gate=None):
    """``committed_gqa`` followed by the decode layer's gating of the read,
    in one launch: ``(read * valid[b]) * head_gate[b, h]`` with each product
    rounded to the query dtype (valid bool ``[B]``, head_gate float ``[B, H]``;
    None skips either)."""
    nb, g, cap, _, d = _check_state(state)
    if query.ndim != 4 or query.shape[1] != 1 or query.shape[3] != d:
        raise ValueError("query must be [B, 1, H, D] with the memory head dim")
    b, _, h, _ = query.shape
    if h % g:
        raise ValueError("query heads must be a multiple of memory groups")
    if query.dtype != state.keys.dtype:
        raise ValueError("query and memory must share a dtype")
    if valid is not None and valid.shape != (b,):
        raise ValueError("valid must be [B]")
    if head_gate is not None and head_gate.shape != (b, h):
        raise ValueError("head_gate must be [B, H]")
    N.require_device(query, state.keys, indices, valid, head_gate)
    idx = _indices(indices, b)
    if idx is None and nb < b:
        raise ValueError("memory state has fewer rows than the batch")
    q = query.contiguous()
    out = torch.empty_like(q)
    rs = _row_strides(state)
    if valid is None and head_gate is None:
        N.call("yh_anchor_read", q.data_ptr(), state.keys.data_ptr(), state.values.data_ptr(),
               state.positions.data_ptr(), N.ptr(idx), out.data_ptr(), b, h, g, cap, d, nb, rs[0], rs[1], rs[3],
               N.code(q), N.stream_of(q))
        return out
    if valid is None or (valid.dtype == torch.bool and valid.is_contiguous()):
        vd = valid                                   # bool is one byte, 0 / 1
    else:
        vd = valid.to(torch.uint8).contiguous()
    hg = None if head_gate is None else head_gate.to(torch.float32).contiguous()
    N.call("yh_anchor_read_gated", q.data_ptr(), state.keys.data_ptr(), state.values.data_ptr(),
           state.positions.data_ptr(), N.ptr(idx), out.data_ptr(), b, h, g, cap, d, nb, rs[0], rs[1], rs[3],
           N.ptr(vd), N.ptr(hg), N.code(q), N.stream_of(q))
    return out


def _batch_rows(t):
    """t [B, 1, G, D] as it is when its heads are contiguous and its batch rows
    keep 16-byte alignment (e.g. the value half of a fused k/v projection),
    a contiguous copy otherwise."""
    _, _, g, d = t.shape
    if t.stride(3) == 1 and t.stride(2) == d and t.stride(0) >= g * d and \
            (t.stride(0) * t.element_size()) % 16 == 0 and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def commit_decode(key, value, scores, active, chunk, state: IndependentMemoryState, indices=None):
    """Push one token per active row into the pending chunk and, when that
    fills the chunk, keep the Top-K_cap of committed + pending slots (score
    descending, then position, then candidate index).  IN PLACE on ``state``.

    key, value ``[B, 1, G, D]``; scores ``[B, 1, G]`` float32; active ``[B]``
    bool."""
    nb, g, cap, pc, d = _check_state(state)
    b = key.shape[0]
    if key.shape != (b, 1, g, d) or value.shape != key.shape:
        raise ValueError("key/value must be [B, 1, G, D]")
    if scores.shape != (b, 1, g):
        raise ValueError("scores must be [B, 1, G]")
    if active.shape != (b,):
        raise ValueError("active must be [B]")
    if not 1 <= int(chunk) <= pc:
        raise ValueError(f"chunk {chunk} must lie in [1, {pc}]")
    if key.dtype != state.keys.dtype or value.dtype != state.keys.dtype:
        raise ValueError("key/value must match the memory dtype")
    N.require_device(key, value, scores, active, state.keys, indices)
    idx = _indices(indices, b)
    if idx is None and nb < b:
        raise ValueError("memory state has fewer rows than the batch")
    k, v = _batch_rows(key), _batch_rows(value)
    sc = scores.to(torch.float32).contiguous()
    act = active.to(torch.bool).contiguous()
    rs = (ctypes.c_int64 * 9)(*_row_strides(state))
    N.call("yh_anchor_commit", k.data_ptr(), v.data_ptr(), sc.data_ptr(), act.data_ptr(), N.ptr(idx),
           state.keys.data_ptr(), state.values.data_ptr(), state.scores.data_ptr(),
           state.positions.data_ptr(), state.pending_keys.data_ptr(), state.pending_values.data_ptr(),
           state.pending_scores.data_ptr(), state.count.data_ptr(), state.total.data_ptr(), b, g, cap, pc,
           int(chunk), d, nb, rs, k.stride(0), v.stride(0), N.code(k), N.stream_of(k))


def sequence(query, key, value, scores, valid, chunk, state: IndependentMemoryState):
    """The anchor-memory read and write of a prefill chunk that continues
    ``state``: IndependentGQAMemory._sequence with a state
    (modeling_yanchor.py:178-275), IN PLACE on ``state``.

    query ``[B, L, H, D]`` (normed, rotated); key, value ``[B, L, G, D]`` the
    written key / value of every token (the reference computes them only for
    the tokens that ever enter the memory; the others are never read);
    scores ``[B, L, G]`` admission scores; valid ``None`` or bool ``[B, L]``
    (valid tokens of a row are taken in order, as the reference's stable
    argsort packs them).  Returns the memory read ``[B, L, H, D]``, zero at
    invalid tokens.  Every token reads the memory committed before its block
    (the old pending tokens open the first block), exactly what a
    token-by-token ``committed_gqa`` / ``commit_decode`` sequence reads, and
    the state ends as that sequence leaves it (slots that hold no token are
    zeroed, as the reference's masked copies do)."""
    nb, g, cap, pc, d = _check_state(state)
    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("query must be [B, L, H, D] and key/value [B, L, G, D]")
    b, length, h, qd = query.shape
    if key.shape != (b, length, g, d) or value.shape != key.shape or qd != d:
        raise ValueError("key/value must be [B, L, G, D] matching the memory")
    if scores.shape != (b, length, g):
        raise ValueError("scores must be [B, L, G]")
    if nb != b:
        raise ValueError("the memory state must have one row per batch row")
    if valid is not None and valid.shape != (b, length):
        raise ValueError("valid must be [B, L]")
    c = int(chunk)
    if not 1 <= c <= pc:
        raise ValueError(f"chunk {chunk} must lie in [1, {pc}]")
    if query.dtype != state.keys.dtype or key.dtype != state.keys.dtype or value.dtype != state.keys.dtype:
        raise ValueError("query/key/value must match the memory dtype")
    for f in fields(state):
        if not getattr(state, f.name).is_contiguous():
            raise ValueError(f"memory state field {f.name} must be contiguous")
    N.require_device(query, key, value, scores, valid, state.keys)
    dev = query.device
    bi = torch.arange(b, device=dev)[:, None]
    if valid is None:
        order = None
        q, k, v, sc = query, key, value, scores
        counts = torch.full((b,), length, device=dev, dtype=torch.long)
    else:
        order = valid.long().argsort(dim=1, descending=True, stable=True)
        q, k, v, sc = (x[bi, order] for x in (query, key, value, scores))
        counts = valid.sum(1)
    blocks = -(-length // c) + 1                  # ceil((L + C) / C) blocks of C positions
    src_k = torch.cat((state.keys.transpose(1, 2), state.pending_keys[:, :, :c].transpose(1, 2), k), 1).contiguous()
    src_v = torch.cat((state.values.transpose(1, 2), state.pending_values[:, :, :c].transpose(1, 2), v),
                      1).contiguous()
    n_src = cap + c + length
    block_refs = torch.empty(b, blocks, g, cap, device=dev, dtype=torch.int32)
    final_refs = torch.empty(b, g, cap, device=dev, dtype=torch.int32)
    pending_refs = torch.empty(b, g, pc, device=dev, dtype=torch.int32)
    sc = sc.to(torch.float32).contiguous()
    counts = counts.to(torch.long).contiguous()
    st = N.stream_of(query)
    N.call("yh_anchor_prefix", sc.data_ptr(), counts.data_ptr(), state.scores.data_ptr(),
           state.positions.data_ptr(), state.pending_scores.data_ptr(), state.count.data_ptr(),
           state.total.data_ptr(), block_refs.data_ptr(), final_refs.data_ptr(), pending_refs.data_ptr(), b, length,
           g, cap, pc, c, blocks, st)
    # block position p of row b reads token p - old[b] in place (the old
    # pending tokens open the first block and read nothing here)
    first = state.count.contiguous()
    qc = q.contiguous()
    out = torch.empty_like(qc)
    N.call("yh_anchor_sequence_read", qc.data_ptr(), src_k.data_ptr(), src_v.data_ptr(), block_refs.data_ptr(),
           N.I32, first.data_ptr(), out.data_ptr(), b, length, blocks, c, h, g, d, n_src, cap, N.code(qc), st)
    if order is not None:
        out = out[bi, order.argsort(1)] * valid[..., None, None].to(out.dtype)
    N.call("yh_anchor_sequence_commit", src_k.data_ptr(), src_v.data_ptr(), final_refs.data_ptr(),
           pending_refs.data_ptr(), counts.data_ptr(), state.keys.data_ptr(), state.values.data_ptr(),
           state.pending_keys.data_ptr(), state.pending_values.data_ptr(), state.count.data_ptr(),
           state.total.data_ptr(), b, n_src, length, g, cap, pc, c, d, N.code(src_k), st)
    return out


def ring_decode_attention(query, keys, values, positions, indices=None, gate=None):
    """Decode attention of one token over a physical ring of cached K/V slots
    (fixed_memory_physical_ring_decode_attention, reference runtime/model/
    inference_kernels.py:1881-1898, on the ring set up at 555-640): softmax
    over the live slots (positions >= 0) without the anchor sink.  query
    [B, 1, H, D]; keys/values [NB, G, window, D]; positions int32
    [NB, G, window].  With ``gate``
    ([B, H, D], any token / head strides, unit last stride) the output is
    ``read * sigmoid(gate)`` (the gated-q output, products rounded to the
    dtype) in the same launch."""
    nb, g, window, d = keys.shape
    if values.shape != keys.shape or positions.shape != (nb, g, window) or positions.dtype != torch.int32:
        raise ValueError("ring keys/values must be [NB, G, W, D] with int32 positions [NB, G, W]")
    if query.ndim != 4 or query.shape[1] != 1 or query.shape[3] != d or query.dtype != keys.dtype:
        raise ValueError("query must be [B, 1, H, D] in the cache dtype")
    b, _, h, _ = query.shape
    N.require_device(query, keys, values, positions, indices, gate)
    for t in (keys, values, positions):
        if not t.is_contiguous():
            raise ValueError("ring tensors must be contiguous")
    idx = _indices(indices, b)
    if idx is None and nb < b:
        raise ValueError("ring has fewer rows than the batch")
    q = query.contiguous()
    out = torch.empty_like(q)
    if gate is None:
        N.call("yh_window_attend", q.data_ptr(), keys.data_ptr(), values.data_ptr(), positions.data_ptr(),
               N.ptr(idx), out.data_ptr(), b, h, g, window, d, nb, N.code(q), N.stream_of(q))
        return out
    if gate.shape != (b, h, d) or gate.stride(-1) != 1 or gate.dtype != q.dtype:
        raise ValueError("gate must be [B, H, D] in the query dtype with unit last stride")
    N.call("yh_window_attend_gated", q.data_ptr(), keys.data_ptr(), values.data_ptr(), positions.data_ptr(),
           N.ptr(idx), out.data_ptr(), b, h, g, window, d, nb, gate.data_ptr(), gate.stride(0), gate.stride(1),
           N.code(q), N.stream_of(q))
    return out
