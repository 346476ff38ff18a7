"""Pins for oracle.gdn that do not retype its formulas.

* closed forms: one step from a zero state; beta = 0 (pure decay);
* invariant: beta = 1 with unit k overwrites the association (S'^T k = v);
* the chunked form (a different algorithm: WY transform + forward
  substitution) equals the token recurrence for chunk sizes 16/32/64, with
  lengths that are and are not multiples of the chunk;
* varlen packing equals per-sequence runs and the left-padded batch with a
  zero state (the reference's padding rule, modeling_yanchor.py:385-390);
* a planted mistake (a dropped decay) is caught by the closed form.
"""
import math

import pytest
import torch

from oracle import gdn
from yanchor_amd import workloads

from conftest import rel_err


def _rand(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def test_single_step_closed_form():
    b, h, kd, vd = 2, 3, 8, 5
    q, k = _rand((b, 1, h, kd), 1), _rand((b, 1, h, kd), 2)
    v = _rand((b, 1, h, vd), 3)
    beta = torch.sigmoid(_rand((b, 1, h), 4))
    g = -torch.rand(b, 1, h, dtype=torch.float64)
    o, s = gdn.recurrent_gated_delta_rule(q, k, v, g, beta)
    qn = q / q.norm(dim=-1, keepdim=True)
    kn = k / k.norm(dim=-1, keepdim=True)
    # S1 = k (beta v)^T ; o = beta (q.k)/sqrt(K) v   (decay of a zero state is irrelevant)
    s_ref = kn[:, 0, :, :, None] * (beta[:, 0, :, None, None] * v[:, 0, :, None, :])
    o_ref = (beta[:, 0] * (qn[:, 0] * kn[:, 0]).sum(-1) / math.sqrt(kd))[..., None] * v[:, 0]
    assert torch.allclose(s, s_ref, atol=1e-6, rtol=1e-6)  # eps=1e-6 inside rsqrt
    assert torch.allclose(o[:, 0], o_ref, atol=1e-6, rtol=1e-6)


def test_zero_beta_is_pure_decay():
    b, t, h, kd, vd = 1, 7, 2, 6, 4
    q, k, v = _rand((b, t, h, kd), 5), _rand((b, t, h, kd), 6), _rand((b, t, h, vd), 7)
    g = -torch.rand(b, t, h, dtype=torch.float64)
    s0 = _rand((b, h, kd, vd), 8)
    o, s = gdn.recurrent_gated_delta_rule(q, k, v, g, torch.zeros(b, t, h, dtype=torch.float64), s0,
                                          use_qk_l2norm=False)
    total = g.sum(1).exp()
    assert torch.allclose(s, s0 * total[..., None, None], atol=1e-12)
    cum = g.cumsum(1).exp()  # state at step i is exp(sum_{<=i} g) S0
    o_ref = torch.einsum("bhkv,bthk->bthv", s0, q / math.sqrt(kd)) * cum[..., None]
    assert torch.allclose(o, o_ref, atol=1e-12)


def test_delta_rule_overwrites_association():
    b, h, kd, vd = 2, 2, 16, 8
    s0 = _rand((b, h, kd, vd), 9)
    q, k, v = _rand((b, 1, h, kd), 10), _rand((b, 1, h, kd), 11), _rand((b, 1, h, vd), 12)
    g = torch.zeros(b, 1, h, dtype=torch.float64)
    one = torch.ones(b, 1, h, dtype=torch.float64)
    _, s = gdn.recurrent_gated_delta_rule(q, k, v, g, one, s0)
    kn = gdn.l2norm(k[:, 0])
    recalled = torch.einsum("bhkv,bhk->bhv", s, kn)
    # |k|^2 = 1 - eps/(|k|^2+eps), so the recall is v up to ~1e-7
    assert torch.allclose(recalled, v[:, 0], atol=1e-6)


def test_planted_mistake_is_caught():
    """A recurrence that forgets the decay fails the beta=0 closed form."""
    b, t, h, kd, vd = 1, 4, 1, 4, 4
    s0 = _rand((b, h, kd, vd), 13)
    g = torch.full((b, t, h), -0.5, dtype=torch.float64)
    z = torch.zeros(b, t, h, dtype=torch.float64)
    q, k, v = _rand((b, t, h, kd), 14), _rand((b, t, h, kd), 15), _rand((b, t, h, vd), 16)
    _, good = gdn.recurrent_gated_delta_rule(q, k, v, g, z, s0)
    _, bad = gdn.recurrent_gated_delta_rule(q, k, v, torch.zeros_like(g), z, s0)  # decay dropped
    expect = s0 * math.exp(-0.5 * t)
    assert torch.allclose(good, expect)
    assert not torch.allclose(bad, expect)


@pytest.mark.parametrize("chunk", [16, 32, 64])
@pytest.mark.parametrize("t", [64, 100])
def test_chunk_equals_recurrent(chunk, t):
    x = workloads.gdn_inputs(2, t, 2, 4, 32, 16, dtype=torch.float64, seed=100 + t, state_std=0.1)
    o1, s1 = gdn.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, x.state)
    o2, s2 = gdn.chunk_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, x.state, chunk_size=chunk)
    assert rel_err(o2, o1) < 1e-10
    assert rel_err(s2, s1) < 1e-10


def test_varlen_equals_per_sequence_and_left_padding():
    lens = [5, 17, 1, 30]
    total = sum(lens)
    x = workloads.gdn_inputs(1, total, 2, 2, 16, 8, dtype=torch.float64, seed=7)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    o, finals = gdn.varlen(gdn.recurrent_gated_delta_rule, x.q, x.k, x.v, x.g, x.beta, cu)
    oc, finals_c = gdn.varlen(gdn.chunk_gated_delta_rule, x.q, x.k, x.v, x.g, x.beta, cu,
                              chunk_size=16)
    assert rel_err(oc, o) < 1e-10 and rel_err(finals_c, finals) < 1e-10
    # left-padded batch: padded tokens have k = v = 0 (zeroed hidden states) and
    # the gates of a zero hidden state; from a zero state they change nothing.
    width = max(lens)
    shp = lambda *s: torch.zeros(len(lens), width, *s, dtype=torch.float64)
    q, k, v = shp(2, 16), shp(2, 16), shp(2, 8)
    g, beta = shp(2) - 0.3, shp(2) + 0.5
    for i, n in enumerate(lens):
        s, e = cu[i], cu[i + 1]
        q[i, width - n:], k[i, width - n:], v[i, width - n:] = x.q[0, s:e], x.k[0, s:e], x.v[0, s:e]
        g[i, width - n:], beta[i, width - n:] = x.g[0, s:e], x.beta[0, s:e]
    op, sp = gdn.recurrent_gated_delta_rule(q, k, v, g, beta)
    assert rel_err(sp, finals) < 1e-12
    for i, n in enumerate(lens):
        assert rel_err(op[i, width - n:], o[0, cu[i]:cu[i + 1]]) < 1e-12


def test_gqa_matches_repeated_heads():
    x = workloads.gdn_inputs(1, 9, 2, 4, 16, 8, dtype=torch.float64, seed=3)
    o1, s1 = gdn.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta)
    q, k = (t.repeat_interleave(2, dim=2) for t in (x.q, x.k))
    o2, s2 = gdn.recurrent_gated_delta_rule(q, k, x.v, x.g, x.beta)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_gates_closed_form():
    b = torch.tensor([0.0, 2.0, -3.0])
    a = torch.tensor([0.0, 25.0, -1.0])
    a_log = torch.tensor([0.0, math.log(2.0), 1.0])
    dt = torch.tensor([0.0, 0.0, 0.5])
    beta, g = gdn.gdn_gates(b, a, a_log, dt)
    assert torch.allclose(beta, torch.tensor([0.5, 1 / (1 + math.exp(-2)), 1 / (1 + math.exp(3))],
                                             dtype=torch.float64))
    # softplus(0) = ln 2; above the threshold softplus(x) = x
    expect = torch.tensor([-math.log(2.0), -2.0 * 25.0, -math.e * math.log1p(math.exp(-0.5))],
                          dtype=torch.float64)
    assert torch.allclose(g, expect)
