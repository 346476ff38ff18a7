"""Anchor-memory slot pages: the vLLM wire format of ``IndependentMemoryState``.

vLLM keeps a recurrent layer's per-request state in two page tensors per slot
(vllm_yanchor.py:21-24, 49-64):

* ``values`` [slots, 2 G (K_cap + C) D] in the model dtype, laid out as
  keys | values | pending_keys | pending_values, each [G, width, D];
* ``meta`` [slots, G (2 K_cap + C) + 4] float32, laid out as
  scores [G, K_cap] | positions [G, K_cap] (int32 bits) | pending_scores [G, C] |
  count (int64 bits) | total (int64 bits).

``state_view`` returns an ``IndependentMemoryState`` whose fields are views into
those pages (no copy).  The decode kernels take such a state directly, with
``state_indices`` selecting the slots: every field is dense within a slot and
the slot stride is passed to the kernels.
"""
from __future__ import annotations

import torch

from .independent_memory import IndependentMemoryState


def memory_shapes(groups: int, capacity: int, chunk: int, dim: int):
    """Per-slot page shapes ((values,), (meta,)) (vllm_yanchor.py:21-24)."""
    return (2 * groups * (capacity + chunk) * dim,), (groups * (2 * capacity + chunk) + 4,)


def state_view(values: torch.Tensor, meta: torch.Tensor, groups: int, capacity: int, chunk: int,
               dim: int) -> IndependentMemoryState:
    """The slot pages as an ``IndependentMemoryState`` of views
    (vllm_yanchor.py:49-64)."""
    (vw,), (mw,) = memory_shapes(groups, capacity, chunk, dim)
    slots = values.shape[0]
    if values.shape != (slots, vw) or meta.shape != (slots, mw) or meta.dtype != torch.float32:
        raise ValueError(f"pages must be values [slots, {vw}] and float32 meta [slots, {mw}]")
    if values.stride(-1) != 1 or meta.stride(-1) != 1 or mw % 2:
        raise ValueError("page rows must be dense with an even meta width")
    tensors, offset = [], 0
    for width in (capacity, capacity, chunk, chunk):
        size = groups * width * dim
        tensors.append(values[:, offset:offset + size].view(slots, groups, width, dim))
        offset += size
    w = groups * capacity
    scores = meta[:, :w].view(slots, groups, capacity)
    positions = meta[:, w:2 * w].view(torch.int32).view(slots, groups, capacity)
    pending_scores = meta[:, 2 * w:-4].view(slots, groups, chunk)
    count = meta[:, -4:-2].view(torch.int64).squeeze(-1)
    total = meta[:, -2:].view(torch.int64).squeeze(-1)
    return IndependentMemoryState(tensors[0], tensors[1], scores, positions, tensors[2], tensors[3], pending_scores,
                                  count, total)


def empty_pages(slots: int, groups: int, capacity: int, chunk: int, dim: int, device, dtype):
    """Pages holding ``slots`` empty memories (scores -inf, positions -1,
    counters 0), as ``IndependentMemoryState.empty`` would."""
    (vw,), (mw,) = memory_shapes(groups, capacity, chunk, dim)
    values = torch.zeros(slots, vw, device=device, dtype=dtype)
    meta = torch.zeros(slots, mw, device=device, dtype=torch.float32)
    state_view(values, meta, groups, capacity, chunk, dim).reset_()
    return values, meta


def page_bytes(groups: int, capacity: int, chunk: int, dim: int, dtype=torch.bfloat16) -> int:
    """Bytes of one slot's pages."""
    (vw,), (mw,) = memory_shapes(groups, capacity, chunk, dim)
    return vw * torch.empty((), dtype=dtype).element_size() + mw * 4


__all__ = ["memory_shapes", "state_view", "empty_pages", "page_bytes"]
