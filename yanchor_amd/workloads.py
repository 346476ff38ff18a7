"""Seeded synthetic inputs for the hot-path workloads.

Inputs are generated on the CPU with ``torch.Generator`` so a CPU run and a GPU
run see identical tensors (copy to the device afterwards).  Distributions:

* q, k ~ N(0, 1), L2-normalised per head; v ~ N(0, 1)
* beta = sigmoid(N(0, 1)); g = logsigmoid(N(0, 1) + 3), per head per token
* recurrent state zeros or ~ N(0, state_std)
* anchor keys / values ~ N(0, 1); each slot live with probability p_live
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

SEED0 = 20260923  # base seed; workload i uses SEED0 + i


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(int(seed))


def _unit(x: torch.Tensor) -> torch.Tensor:
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)


@dataclass
class GdnInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    g: torch.Tensor
    beta: torch.Tensor
    state: torch.Tensor
    state_indices: torch.Tensor | None

    def to(self, device) -> "GdnInputs":
        return GdnInputs(*(None if x is None else x.to(device) for x in
                           (self.q, self.k, self.v, self.g, self.beta, self.state,
                            self.state_indices)))


def gdn_inputs(B, T, H, HV, K, V, *, dtype=torch.float32, seed=SEED0, state_std=0.0,
               pool_rows=None, gate_dtype=torch.float32) -> GdnInputs:
    """Token inputs [B, T, ...] plus a float32 state pool.

    With ``pool_rows`` (> B) the state is a slot pool of that many rows and the
    batch rows map to a seeded random subset of slots (``state_indices``), the
    ragged live-slot layout of a continuous batch.
    """
    gen = _gen(seed)
    q = _unit(torch.randn(B, T, H, K, generator=gen))
    k = _unit(torch.randn(B, T, H, K, generator=gen))
    v = torch.randn(B, T, HV, V, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, HV, generator=gen))
    g = F.logsigmoid(torch.randn(B, T, HV, generator=gen) + 3.0)
    rows = B if pool_rows is None else int(pool_rows)
    if state_std:
        state = torch.randn(rows, HV, K, V, generator=gen) * state_std
    else:
        state = torch.zeros(rows, HV, K, V)
    idx = None
    if pool_rows is not None:
        idx = torch.randperm(rows, generator=gen)[:B].to(torch.int32)
    return GdnInputs(q.to(dtype), k.to(dtype), v.to(dtype), g.to(gate_dtype), beta.to(gate_dtype),
                     state, idx)


def cpu_gdn_config0() -> GdnInputs:
    """CPU reference recurrence: B=2, T=256, H=4, dk=dv=64, fp32, zero state."""
    return gdn_inputs(2, 256, 4, 4, 64, 64, dtype=torch.float32, seed=SEED0 + 0)


def decode_gdn_config1(pool_rows: int = 96) -> GdnInputs:
    """Decode step: 64 live rows of a slot pool, HV=32, dk=dv=128, state ~ N(0, 0.02),
    q/k/v bf16, g/beta fp32."""
    return gdn_inputs(64, 1, 32, 32, 128, 128, dtype=torch.bfloat16, seed=SEED0 + 1,
                      state_std=0.02, pool_rows=pool_rows)


def anchor_state(B, G, capacity, chunk, D, *, p_live=0.7, seed=SEED0 + 1, dtype=torch.bfloat16,
                 fill_pending=0, total0=None):
    """Anchor memory state on the CPU: keys/values ~ N(0, 1); slot n of (b, g)
    live with probability p_live (position >= 0, score ~ N(0, 1)), dead slots
    carry position -1 and score -inf.  ``fill_pending`` pending entries are
    already pushed (count = fill_pending) and total = total0 (default
    4 * capacity + fill_pending, past the largest committed position)."""
    from .independent_memory import IndependentMemoryState
    gen = _gen(seed)
    st = IndependentMemoryState.empty(B, G, capacity, chunk, D, "cpu", dtype)
    st.keys.copy_(torch.randn(B, G, capacity, D, generator=gen).to(dtype))
    st.values.copy_(torch.randn(B, G, capacity, D, generator=gen).to(dtype))
    live = torch.rand(B, G, capacity, generator=gen) < p_live
    pos = torch.randperm(capacity * 4, generator=gen)[:capacity].sort().values.to(torch.int32)
    st.positions.copy_(torch.where(live, pos.expand(B, G, capacity), torch.tensor(-1, dtype=torch.int32)))
    sc = torch.randn(B, G, capacity, generator=gen)
    st.scores.copy_(torch.where(live, sc, torch.tensor(-float("inf"))))
    if fill_pending:
        st.pending_keys[:, :, :fill_pending] = torch.randn(B, G, fill_pending, D, generator=gen).to(dtype)
        st.pending_values[:, :, :fill_pending] = torch.randn(B, G, fill_pending, D, generator=gen).to(dtype)
        st.pending_scores[:, :, :fill_pending] = torch.randn(B, G, fill_pending, generator=gen)
    st.count.fill_(fill_pending)
    st.total.fill_(capacity * 4 + fill_pending if total0 is None else total0)
    return st


def anchor_query(B, H, D, *, seed=SEED0 + 2, dtype=torch.bfloat16):
    return torch.randn(B, 1, H, D, generator=_gen(seed)).to(dtype)


@dataclass
class PackedInputs:
    q: torch.Tensor        # [1, total, H, K]
    k: torch.Tensor
    v: torch.Tensor        # [1, total, HV, V]
    g: torch.Tensor        # [1, total, HV]
    beta: torch.Tensor
    cu_seqlens: torch.Tensor  # int32 [N + 1]
    lengths: list
    h0: torch.Tensor | None

    def to(self, device) -> "PackedInputs":
        return PackedInputs(*(x.to(device) for x in (self.q, self.k, self.v, self.g, self.beta,
                                                       self.cu_seqlens)),
                            self.lengths, None if self.h0 is None else self.h0.to(device))


def prefill_lengths(n=32, lo=512, hi=8192, seed=SEED0 + 2):
    """Sequence lengths uniform in [lo, hi] (seeded)."""
    return torch.randint(lo, hi + 1, (n,), generator=_gen(seed)).tolist()


def packed_inputs(lengths, H, HV, K, V, *, dtype=torch.bfloat16, seed=SEED0 + 2, h0_std=0.0):
    """Packed varlen inputs with the distributions of the module docstring."""
    gen = _gen(seed)
    total = int(sum(lengths))
    q = _unit(torch.randn(1, total, H, K, generator=gen))
    k = _unit(torch.randn(1, total, H, K, generator=gen))
    v = torch.randn(1, total, HV, V, generator=gen)
    beta = torch.sigmoid(torch.randn(1, total, HV, generator=gen))
    g = F.logsigmoid(torch.randn(1, total, HV, generator=gen) + 3.0)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.int32)
    h0 = torch.randn(len(lengths), HV, K, V, generator=gen) * h0_std if h0_std else None
    return PackedInputs(q.to(dtype), k.to(dtype), v.to(dtype), g, beta, cu, list(lengths), h0)
