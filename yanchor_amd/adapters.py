"""The anchor-memory layer of the vLLM and SGLang model adapters on ROCm.

The reference's adapters run the memory branch of a YANchor decoder layer on
the serving framework's per-request state, and disable their CUDA path on
ROCm (``torch.version.hip`` checks at vllm_yanchor.py:34, 155 and
sglang_models/yanchor.py:48, 134).  Here the same layer forward runs on the
HIP kernels:

* ``VllmMemory.forward(hidden [N, hidden], positions [N])``
  (vllm_yanchor.py:66-97): the metadata comes from the forward context under
  the layer's prefix and the slot pages (the wire format of ``slot_pages``)
  from the bound ``kv_cache``.  The first ``num_decodes`` tokens are one
  decode token each, read and committed in place on the pages with
  ``state_indices`` (negative = padding, skipped); every later request is a
  prefill span of ``non_spec_query_start_loc``: its slot is read out, reset
  when the span starts at position 0, continued by the block-wise prefill
  read / write (``_sequence`` with a state), and written back.
* ``MemorySlots`` + ``SglangMemory.forward(hidden, positions, forward_batch)``
  (sglang_models/yanchor.py:18-83): the same over an
  ``IndependentMemoryState`` of size + 1 rows with the slot lifecycle
  ``reset_slots`` / ``copy_slots`` / ``get_cpu_slots`` / ``load_cpu_slots``;
  a decode batch runs in place on the request rows, an extend batch request
  by request (reset when its prefix length is 0).

Neither serving framework is importable here, so each layer also takes the
framework's getter (vLLM's ``get_forward_context``, SGLang's
``get_req_to_token_pool``) as a constructor argument.

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


def _text_positions(positions):
    """Token positions [N] of a call; vLLM and SGLang may hand the three
    M-RoPE rows [3, N], which coincide for text tokens (the reference expands
    a 1-D tensor to exactly that, vllm_yanchor.py:68)."""
    return positions[0] if positions.ndim == 2 else positions


class VllmMemory(MemoryLayer):
    """YANchorMemory of vllm_yanchor.py:21-97 on the slot pages.

    ``forward(hidden, positions)`` is the reference layer's call: the batch's
    GDN attention metadata is read from the forward context under the layer's
    ``prefix`` (``get_forward_context().attn_metadata[prefix]``; vLLM's own
    getter when vLLM is importable, else the ``forward_context`` callable given
    here), and the slot pages from ``kv_cache`` = ``(values, meta)``, which the
    caller binds as vLLM binds a Mamba-type layer's cache.  With no metadata
    (vLLM's profiling and dummy runs) the batch is one sequence over a fresh
    memory and no page is touched.  ``run`` is the same forward with the
    metadata and pages passed explicitly."""

    def __init__(self, model: rt.Model, layer: int, prefix: str = "", forward_context=None):
        super().__init__(model, layer)
        self.prefix = prefix
        self._forward_context = forward_context
        self.kv_cache = None

    @property
    def state_shapes(self):
        c = self.cfg
        return slot_pages.memory_shapes(c.kv_heads, c.memory_capacity, self.chunk, c.head_dim)

    def get_state_shape(self):
        return self.state_shapes

    def get_state_dtype(self):
        return (self.m.dtype, torch.float32)

    def get_forward_context(self):
        if self._forward_context is not None:
            return self._forward_context()
        try:
            from vllm.forward_context import get_forward_context
        except ImportError:
            raise RuntimeError("VllmMemory.forward needs a forward context: vLLM is not importable here, so "
                               "pass forward_context= (a callable returning an object with attn_metadata)") from None
        return get_forward_context()

    def state(self, pages=None):
        values, meta = self.kv_cache if pages is None else pages
        c = self.cfg
        return slot_pages.state_view(values, meta, c.kv_heads, c.memory_capacity, self.chunk, c.head_dim)

    def forward(self, hidden, positions):
        """Memory branch output [N, hidden] of the batch's tokens
        (vllm_yanchor.py:66-97); the bound pages are updated in place."""
        positions = _text_positions(positions)
        metadata = self.get_forward_context().attn_metadata
        if metadata is None:
            return self.run_fresh(hidden, positions)
        if self.kv_cache is None:
            raise RuntimeError(f"VllmMemory {self.prefix!r}: no kv_cache (values, meta) pages bound")
        return self.run(hidden, positions, metadata[self.prefix], self.kv_cache)

    def run_fresh(self, hidden, positions):
        """The batch as one sequence over an empty memory, as the reference
        layer runs without a cache."""
        c = self.cfg
        state = im.IndependentMemoryState.empty(1, c.kv_heads, c.memory_capacity, self.chunk, c.head_dim,
                                                hidden.device, hidden.dtype)
        q, gate, key, value, scores = self.project_sequence(hidden, positions)
        return self.output(self.memory_sequence(q, key, value, scores, state)[0], gate[0])

    def run(self, hidden, positions, metadata: VllmMetadata, pages, return_reads=False):
        """Memory branch output [N, hidden] for the batch's tokens with the
        metadata and pages given; the pages are updated in place."""
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
    """YANchorMemory of sglang_models/yanchor.py:42-83 on ``MemorySlots``.

    ``forward(hidden, positions, forward_batch)`` is the reference layer's
    call.  The request-to-token pool comes from SGLang's
    ``get_req_to_token_pool()`` when SGLang is importable, else from the
    ``req_to_token_pool`` callable given here; on the first call the layer
    creates its ``MemorySlots`` with the pool's mamba pool size and registers
    them with ``register_slot_state``.  The request rows are
    ``translate_mamba_indices(get_mamba_indices(forward_batch.req_pool_indices))``;
    ``forward_batch.forward_mode.is_decode()`` selects the decode path, else
    the extend spans of ``extend_seq_lens_cpu`` run request by request, a
    request whose ``extend_prefix_lens_cpu`` is 0 starting from an empty
    memory.  ``run`` is the same forward with the slots and rows passed
    explicitly."""

    def __init__(self, model: rt.Model, layer: int, layer_id: int | None = None, req_to_token_pool=None):
        super().__init__(model, layer)
        self.layer_id = layer if layer_id is None else layer_id
        self._req_to_token_pool = req_to_token_pool
        self.slots = None

    def get_req_to_token_pool(self):
        if self._req_to_token_pool is not None:
            return self._req_to_token_pool()
        try:
            from sglang.srt.model_executor.forward_context import get_req_to_token_pool
        except ImportError:
            raise RuntimeError("SglangMemory.forward needs the request-to-token pool: SGLang is not importable "
                               "here, so pass req_to_token_pool= (a callable returning the pool)") from None
        return get_req_to_token_pool()

    def forward(self, hidden, positions, forward_batch):
        """Memory branch output [N, hidden] (sglang_models/yanchor.py:53-83);
        the request rows of the slots are updated in place."""
        requests = self.get_req_to_token_pool()
        pool = requests.mamba_pool
        if self.slots is None:
            self.slots = MemorySlots(self, pool.size, hidden.device, hidden.dtype, self.layer_id)
            pool.register_slot_state(self.slots)
        indices = requests.translate_mamba_indices(requests.get_mamba_indices(forward_batch.req_pool_indices))
        if forward_batch.forward_mode.is_decode():
            return self.run(hidden, positions, self.slots, indices, decode=True)
        return self.run(hidden, positions, self.slots, indices, decode=False,
                        extend_seq_lens=forward_batch.extend_seq_lens_cpu,
                        extend_prefix_lens=forward_batch.extend_prefix_lens_cpu)

    def run(self, hidden, positions, slots: MemorySlots, indices, *, decode: bool, extend_seq_lens=None,
            extend_prefix_lens=None):
        """Decode: one token per request, in place on the request rows.
        Extend: request spans of ``extend_seq_lens`` (host ints); a request
        whose ``extend_prefix_lens`` is 0 starts from an empty memory."""
        positions = _text_positions(positions)
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
