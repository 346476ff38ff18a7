"""The anchor-memory layer of the vLLM and SGLang model adapters on ROCm.

The reference's adapters run the memory branch of a YANchor decoder layer on
the serving framework's per-request state, and disable their CUDA path on
ROCm (``torch.version.hip`` checks at vllm_yanchor.py:34, 155 and
sglang_models/yanchor.py:48, 134).  Here the same layer forward runs on the
HIP kernels:

* ``VllmMemory.forward(hidden [N, hidden], positions [N], metadata, pages)``
  (vllm_yanchor.py:66-97): the first ``num_decodes`` tokens are one decode
  token each, read and committed in place on the slot pages (the wire format
  of ``slot_pages``) with ``state_indices`` (negative = padding, skipped);
  every later request is a prefill span of ``non_spec_query_start_loc``: its
  slot is read out, reset when the span starts at position 0, continued by
  the block-wise prefill read / write (``_sequence`` with a state), and written
  back.
* ``MemorySlots`` + ``SglangMemory.forward(hidden, positions, slots,
  indices, ...)`` (sglang_models/yanchor.py:18-83): the same over an
  ``IndependentMemoryState`` of size + 1 rows with the slot lifecycle
  ``reset_slots`` / ``copy_slots`` / ``get_cpu_slots`` / ``load_cpu_slots``;
  a decode batch runs in place with the request indices, an extend batch
  request by request (reset when its prefix length is 0).

The weights are those of one attention layer of a ``runtime.Model`` (the
memory's input norm, fused q / admission / writer projection, k / v, output
projection).  ``project_*`` and ``memory_*`` are separate steps, so a caller
(or a test) can run the memory operations on given projections.
"""
from __future__ import annotations

from dataclasses import dataclass, fields

import torch
import torch.nn.functional as F

from . import independent_memory as im
from . import runtime as rt
from . import slot_pages


@dataclass
class VllmMetadata:
    """The fields of vLLM's GDN attention metadata the memory layer reads
    (vllm_yanchor.py:75-86): decode requests first, one token each."""
    num_decodes: int
    num_prefills: int
    non_spec_state_indices_tensor: torch.Tensor   # [requests] int, negative = padding
    non_spec_query_start_loc: torch.Tensor        # [requests + 1] int token offsets


class MemoryLayer:
    """The anchor-memory branch of attention layer ``layer`` of ``model``."""

    def __init__(self, model: rt.Model, layer: int):
        if model.layers[layer]["kind"] != "attn":
            raise ValueError(f"layer {layer} is not an attention / memory layer")
        self.m, self.L, self.cfg = model, model.layers[layer], model.cfg
        self.chunk = min(self.cfg.memory_chunk, self.cfg.swa_window)

    # ---------------- projections ----------------
    def project_decode(self, hidden, positions):
        """(q [N, H, D], gate [N, H], key / value [N, G, D], scores [N, G]) of
        one decode token per row (_query_scores + _write_kv)."""
        cos, sin = rt.rope_tables(positions, self.cfg)
        return self.m._memory_decode(self.L, hidden, cos, sin)

    def project_sequence(self, hidden, positions):
        """The same for one request's span: hidden [L, hidden] ->
        q [1, L, H, D], gate [1, L, H], key / value [1, L, G, D], scores [1, L, G]."""
        cos, sin = rt.rope_tables(positions, self.cfg)
        q, gate, key, value, scores = self.m._memory_qkvs(self.L, hidden[None], cos[None, :, None],
                                                           sin[None, :, None])
        return q.contiguous(), gate, key.contiguous(), value, scores.float()

    # ---------------- memory operations ----------------
    def memory_decode(self, q, gate, key, value, scores, state, indices):
        """Gated read of the committed slots, then push + commit, in place on
        ``state`` rows ``indices`` ([N] int, negative = skip)."""
        valid = indices >= 0
        read = im.committed_gqa_gated(q[:, None], state, indices, valid, gate)
        im.commit_decode(key[:, None], value[:, None], scores[:, None], valid, self.chunk, state, indices)
        return read[:, 0]

    def memory_sequence(self, q, key, value, scores, state):
        """Block-wise prefill read / write continuing ``state`` (one row)."""
        return im.sequence(q, key, value, scores, None, self.chunk, state)

    def output(self, read, gate):
        """o_proj(read * gate) of [..., H, D] reads (the decode read comes
        gated already: pass gate=None)."""
        if gate is not None:
            read = read * gate[..., None].to(read.dtype)
        return F.linear(read.flatten(-2), self.L["m_o"])


class VllmMemory(MemoryLayer):
    """YANchorMemory of vllm_yanchor.py on the slot pages."""

    @property
    def state_shapes(self):
        c = self.cfg
        return slot_pages.memory_shapes(c.kv_heads, c.memory_capacity, self.chunk, c.head_dim)

    def state(self, pages):
        values, meta = pages
        c = self.cfg
        return slot_pages.state_view(values, meta, c.kv_heads, c.memory_capacity, self.chunk, c.head_dim)

    def forward(self, hidden, positions, metadata: VllmMetadata, pages, return_reads=False):
        """Memory branch output [N, hidden] for the batch's tokens; the pages
        are updated in place."""
        pool = self.state(pages)
        indices = metadata.non_spec_state_indices_tensor.to(hidden.device).long()
        out = torch.empty_like(hidden)
        reads = torch.zeros(hidden.shape[0], self.cfg.attn_heads, self.cfg.head_dim, device=hidden.device,
                            dtype=hidden.dtype) if return_reads else None
        n = int(metadata.num_decodes)
        if n:
            q, gate, key, value, scores = self.project_decode(hidden[:n], positions[:n])
            read = self.memory_decode(q, gate, key, value, scores, pool, indices[:n])
            out[:n] = self.output(read, None)
            if return_reads:
                reads[:n] = read
        starts = metadata.non_spec_query_start_loc.tolist() if metadata.num_prefills else []
        for i in range(n, len(starts) - 1):
            lo, hi = starts[i], starts[i + 1]
            if hi == lo:
                continue
            row = indices[i:i + 1]
            state = pool.select(row)
            if int(positions[lo]) == 0:
                state.reset_()
            q, gate, key, value, scores = self.project_sequence(hidden[lo:hi], positions[lo:hi])
            read = self.memory_sequence(q, key, value, scores, state)[0]
            out[lo:hi] = self.output(read, gate[0])
            if return_reads:
                reads[lo:hi] = read * gate[0][..., None].to(read.dtype)
            pool.scatter_(state, row, torch.zeros(1, dtype=torch.long, device=hidden.device))
        return (out, reads) if return_reads else out


class MemorySlots:
    """Per-request anchor-memory rows of one layer for SGLang's pool
    (sglang_models/yanchor.py:18-40): ``size + 1`` rows, the last one the
    pool's padding row."""

    def __init__(self, layer: MemoryLayer, size: int, device, dtype, layer_id: int):
        c = layer.cfg
        self.state = im.IndependentMemoryState.empty(size + 1, c.kv_heads, c.memory_capacity, layer.chunk,
                                                     c.head_dim, device, dtype)
        self.layer_id = layer_id

    def reset_slots(self, indices):
        self.state.reset_(indices.long())

    def copy_slots(self, src_index, dst_index):
        self.state.scatter_(self.state, dst_index.long(), src_index.long())

    def get_cpu_slots(self, indices):
        idx = indices.long().to(self.state.keys.device)
        return {f.name: getattr(self.state, f.name).index_select(0, idx).cpu() for f in fields(self.state)}

    def load_cpu_slots(self, data, indices):
        idx = indices.long().to(self.state.keys.device)
        for name, value in data.items():
            target = getattr(self.state, name)
            target.index_copy_(0, idx, value.to(target.device))

    def iter_transfer_state_entries(self):
        for f in fields(self.state):
            yield f"yanchor_{f.name}", getattr(self.state, f.name), None, self.layer_id


class SglangMemory(MemoryLayer):
    """YANchorMemory of sglang_models/yanchor.py on ``MemorySlots``."""

    def forward(self, hidden, positions, slots: MemorySlots, indices, *, decode: bool, extend_seq_lens=None,
                extend_prefix_lens=None):
        """Decode: one token per request, in place on the request rows.
        Extend: request spans of ``extend_seq_lens`` (host ints); a request
        whose ``extend_prefix_lens`` is 0 starts from an empty memory."""
        indices = indices.to(hidden.device).long()
        if decode:
            q, gate, key, value, scores = self.project_decode(hidden, positions)
            return self.output(self.memory_decode(q, gate, key, value, scores, slots.state, indices), None)
        out = torch.empty_like(hidden)
        start = 0
        for row, length in enumerate(extend_seq_lens):
            if not length:
                continue
            idx = indices[row:row + 1]
            state = slots.state.select(idx)
            if extend_prefix_lens[row] == 0:
                state.reset_()
            q, gate, key, value, scores = self.project_sequence(hidden[start:start + length],
                                                                positions[start:start + length])
            read = self.memory_sequence(q, key, value, scores, state)[0]
            out[start:start + length] = self.output(read, gate[0])
            slots.state.scatter_(state, idx, torch.zeros(1, dtype=torch.long, device=hidden.device))
            start += length
        return out


__all__ = ["VllmMetadata", "MemoryLayer", "VllmMemory", "MemorySlots", "SglangMemory"]
