"""Counter-based sampling on the CPU (oracle; test infrastructure only).

Restates runtime/model/inference_kernels.py:

* ``counter_uniform``             24-33  (32-bit PCG-style output hash of the
                                          (attempt id, step, seed, stream) counter)
* ``sample_cdf_counter``          35-40
* ``top_k_top_p_distribution``    42-58
* ``sample_top_k_top_p_counter``  73-88  (with sample_probabilities_counter 60-71)
* ``top20_counter_sample``        1119-1145 (the fused top-20 kernel; its
                                          caller 1147-1167 does torch.topk and /T)
* ``presence_penalty``            1095-1114

Pins (tests/test_oracle_sampling_slots.py): golden vectors written from the
reference's own functions in tests/golden/counter_sampling.npz; integer hash
values checked with numpy
uint32 wrap-around arithmetic (an independent evaluation order); special cases
top_k = 1 -> argmax, top_p = 1 -> plain inverse CDF; the output of the hash is
a permutation-free uniform (mean/variance over 1e5 counters).
"""
from __future__ import annotations

import math

import numpy as np
import torch

MASK = 0xFFFFFFFF


def counter_word(attempt_id: int, step: int, seed: int, stream: int = 0) -> int:
    """The 32-bit hash word (inference_kernels.py:28-32), in Python ints."""
    state = ((attempt_id & MASK) * 747796405 + (step & MASK) * 289133645
             + (seed & MASK) * 277803737 + (stream & MASK) * 144269504) & MASK
    shift = (state >> 28) + 4
    word = (((state >> shift) ^ state) * 277803737) & MASK
    return ((word >> 22) ^ word) & MASK


def counter_uniform(attempt_ids, steps, *, seed: int, stream: int = 0, dtype=torch.float32):
    """u = (word + 0.5) / 2^32 in float64, cast to ``dtype`` and clamped below
    1 by eps/2 (inference_kernels.py:33)."""
    ids = [int(x) for x in torch.as_tensor(attempt_ids).reshape(-1).tolist()]
    st = torch.as_tensor(steps)
    st = [int(st)] * len(ids) if st.ndim == 0 else [int(x) for x in st.reshape(-1).tolist()]
    u = torch.tensor([(counter_word(a, s, seed, stream) + 0.5) / 4294967296.0
                      for a, s in zip(ids, st)], dtype=torch.float64)
    return u.to(dtype).clamp_max(1.0 - torch.finfo(dtype).eps / 2)


def sample_cdf_counter(probabilities, attempt_ids, steps, *, seed, stream=0):
    """Inverse-CDF draw: first index whose cumulative probability reaches
    min(u * total, nextafter(total, 0)) (inference_kernels.py:35-40)."""
    cumulative = probabilities.cumsum(-1)
    total = cumulative[:, -1:]
    u = counter_uniform(attempt_ids, steps, seed=seed, stream=stream, dtype=probabilities.dtype)[:, None]
    threshold = torch.minimum(u * total, torch.nextafter(total, torch.zeros_like(total)))
    return torch.searchsorted(cumulative, threshold, right=False)


def top_k_top_p_distribution(scores, *, temperature, top_k, top_p):
    """(indices, probabilities) of the top-k after temperature, truncated where
    the probability mass before a token reaches top_p, renormalised
    (inference_kernels.py:42-58)."""
    if temperature == 1.0:
        values, indices = torch.topk(scores, top_k, dim=-1)
        values = values.float()
    else:
        values, indices = torch.topk(scores.float() / temperature, top_k, dim=-1)
    p = torch.softmax(values, dim=-1)
    keep = p.cumsum(-1) - p < top_p
    p = p * keep
    return indices, p / p.sum(-1, keepdim=True)


def sample_top_k_top_p_counter(scores, attempt_ids, steps, *, seed, temperature, top_k, top_p,
                               stream=0):
    """Token ids [B, 1] (inference_kernels.py:73-88)."""
    if top_k <= 0 and top_p == 1.0:
        p = torch.softmax(scores.float() / temperature, dim=-1)
        return sample_cdf_counter(p, attempt_ids, steps, seed=seed, stream=stream)
    if top_k == 1:
        return scores.argmax(dim=-1, keepdim=True)
    indices, p = top_k_top_p_distribution(scores, temperature=temperature,
                                          top_k=top_k if top_k > 0 else scores.shape[-1], top_p=top_p)
    p = p / p.sum(-1, keepdim=True)
    ranks = sample_cdf_counter(p, attempt_ids, steps, seed=seed, stream=stream)
    return indices.gather(1, ranks)


def top20_counter_sample(values, indices, attempt_ids, steps, *, seed, top_p):
    """The fused top-20 sampler (inference_kernels.py:1119-1145) on already
    temperature-scaled, descending top-k ``values`` [B, S] with their vocabulary
    ``indices``.  float32 arithmetic in the kernel's order: softmax with the row
    max subtracted, prefix_before = cumsum(p) - p, keep p where
    prefix_before < top_p, threshold = u * retained (u NOT clamped),
    rank = #(cumulative < threshold) capped at S - 1."""
    values = values.float()
    bsz, support = values.shape
    st = torch.as_tensor(steps)
    st = [int(st)] * bsz if st.ndim == 0 else [int(x) for x in st.reshape(-1).tolist()]
    ids = [int(x) for x in torch.as_tensor(attempt_ids).reshape(-1).tolist()]
    out = torch.empty(bsz, 1, dtype=torch.long)
    for b in range(bsz):
        v = values[b]
        w = torch.exp(v - v.max())
        p = w / w.sum()
        before = p.cumsum(0) - p
        trunc = torch.where(before < top_p, p, torch.zeros_like(p))
        retained = trunc.sum()
        cum = trunc.cumsum(0)
        u = torch.tensor((counter_word(ids[b], st[b], seed) + 0.5) / 4294967296.0,
                         dtype=torch.float64).float()
        rank = int((cum < u * retained).sum())
        out[b, 0] = indices[b, min(rank, support - 1)]
    return out


def presence_penalty(scores, seen, penalty):
    """scores - penalty where seen (inference_kernels.py:1095-1114), float32."""
    return scores.float() - torch.where(seen.bool(), torch.tensor(float(penalty)), torch.tensor(0.0))


def counter_words_numpy(attempt_ids, steps, seed, stream=0):
    """Independent uint32 evaluation of the hash with numpy wrap-around
    arithmetic (used to cross-check ``counter_word``)."""
    with np.errstate(over="ignore"):
        a = np.asarray(attempt_ids, dtype=np.int64).astype(np.uint32)
        s = np.asarray(steps, dtype=np.int64).astype(np.uint32)
        st = (a * np.uint32(747796405) + s * np.uint32(289133645)
              + np.uint32(seed & MASK) * np.uint32(277803737)
              + np.uint32(stream & MASK) * np.uint32(144269504)).astype(np.uint32)
        shift = (st >> np.uint32(28)) + np.uint32(4)
        w = ((st >> shift) ^ st) * np.uint32(277803737)
        return (w >> np.uint32(22)) ^ w
