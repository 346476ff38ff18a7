"""GPU parity of the prefill paths (packed varlen) with the oracle.

Small packed batches are checked against the float64 oracle (chunk-form and
recurrent-form agree in float64, tests/test_oracle_gdn.py): bf16 outputs within
2e-2, final states within 1e-3 (Frobenius relative error).  The full prefill
shape (32 sequences, lengths uniform in [512, 8192], H = HV = 32, d = 128)
is too large for the oracle in seconds; there the MFMA chunk kernel is checked
against the token-recurrent kernel -- a different algorithm that is itself
oracle-checked -- to the same tolerances.
"""
import pytest
import torch

from oracle import gdn as ref
from yanchor_amd import gdn, workloads

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _oracle(x):
    return ref.varlen(ref.recurrent_gated_delta_rule, x.q, x.k, x.v, x.g, x.beta, x.cu_seqlens.tolist(),
                      initial_state=x.h0)


@pytest.mark.parametrize("force_recurrent", [False, True])
@pytest.mark.parametrize("lengths,h,hv", [([1, 63, 64, 65, 130, 200, 7], 2, 4), ([300, 0, 64, 129], 4, 4)])
def test_packed_matches_oracle(gpu, force_recurrent, lengths, h, hv):
    x = workloads.packed_inputs(lengths, h, hv, 128, 128, seed=sum(lengths), h0_std=0.05)
    d = x.to(gpu)
    o, st = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, initial_state=d.h0,
                                       output_final_state=True, use_qk_l2norm_in_kernel=True,
                                       cu_seqlens=d.cu_seqlens, lengths=x.lengths,
                                       force_recurrent=force_recurrent)
    torch.cuda.synchronize()
    ro, rs = _oracle(x)
    assert rel_err(o, ro) <= 2e-2, rel_err(o, ro)
    assert rel_err(st, rs) <= 1e-3, rel_err(st, rs)
    assert torch.equal(d.h0.cpu(), x.h0)  # the initial state is read, not modified


def test_packed_zero_state_and_value_tiles(gpu):
    x = workloads.packed_inputs([100, 37], 1, 2, 128, 64, seed=3)
    d = x.to(gpu)
    o, st = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, output_final_state=True,
                                       use_qk_l2norm_in_kernel=True, cu_seqlens=d.cu_seqlens)
    ro, rs = _oracle(x)
    assert rel_err(o, ro) <= 2e-2 and rel_err(st, rs) <= 1e-3


def test_packed_value_tiles_many_chunks(gpu):
    """V = 64 (four-wave workgroups) over sequences of 1 to 5 chunks with GQA:
    the kernel's two LDS buffers alternate several times per sequence."""
    x = workloads.packed_inputs([300, 129, 1, 64, 192], 2, 4, 128, 64, seed=11, h0_std=0.05)
    d = x.to(gpu)
    o, st = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, initial_state=d.h0,
                                       output_final_state=True, use_qk_l2norm_in_kernel=True,
                                       cu_seqlens=d.cu_seqlens, lengths=x.lengths)
    ro, rs = _oracle(x)
    assert rel_err(o, ro) <= 2e-2, rel_err(o, ro)
    assert rel_err(st, rs) <= 1e-3, rel_err(st, rs)


def test_batched_form(gpu):
    x = workloads.gdn_inputs(2, 70, 2, 2, 128, 128, dtype=torch.bfloat16, seed=8, state_std=0.02)
    d = x.to(gpu)
    o, st = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, initial_state=d.state,
                                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    ro, rs = ref.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, x.state)
    assert rel_err(o, ro) <= 2e-2 and rel_err(st, rs) <= 1e-3
    assert torch.equal(d.state.cpu(), x.state)


def test_full_prefill_shape_chunk_vs_recurrent(gpu):
    lengths = workloads.prefill_lengths()
    x = workloads.packed_inputs(lengths, 32, 32, 128, 128, h0_std=0.0)
    d = x.to(gpu)
    kw = dict(g=d.g, beta=d.beta, output_final_state=True, use_qk_l2norm_in_kernel=True,
              cu_seqlens=d.cu_seqlens, lengths=lengths)
    o1, s1 = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, **kw)
    o2, s2 = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, force_recurrent=True, **kw)
    torch.cuda.synchronize()
    assert rel_err(o1, o2) <= 2e-2, rel_err(o1, o2)
    assert rel_err(s1, s2) <= 1e-3, rel_err(s1, s2)


def _heads(x, heads):
    """The inputs of a subset of heads (H == HV): heads are independent."""
    return [t[:, :, heads].contiguous() for t in (x.q, x.k, x.v, x.g, x.beta)]


def test_reference_batched_call_runs_the_chunk_kernel(gpu, monkeypatch):
    """The reference calls chunk_gated_delta_rule batched, without cu_seqlens
    (wheel modeling_qwen3_5.py:519-529).  At [2, 4096, 32, 128] that call runs
    the MFMA chunk kernel (not the token recurrence) and matches the float64
    oracle on three of the heads (heads are independent)."""
    from yanchor_amd import _native
    calls = []
    real = _native.call

    def spy(name, *args):
        calls.append(name)
        return real(name, *args)

    monkeypatch.setattr(gdn.N, "call", spy)
    x = workloads.gdn_inputs(2, 4096, 32, 32, 128, 128, dtype=torch.bfloat16, seed=21, state_std=0.02)
    d = x.to(gpu)
    o, st = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, initial_state=d.state,
                                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert calls == ["yh_gdn_chunk_varlen"], calls
    assert o.shape == (2, 4096, 32, 128) and st.shape == (2, 32, 128, 128)
    assert torch.equal(d.state.cpu(), x.state)            # the initial state is read, not modified
    heads = [0, 17, 31]
    q, k, v, g, beta = _heads(x, heads)
    ro, rs = ref.chunk_gated_delta_rule(q, k, v, g, beta, x.state[:, heads])
    eo, es = rel_err(o[:, :, heads], ro), rel_err(st[:, heads], rs)
    print(f"[2, 4096, 32, 128] heads {heads}: out rel err {eo:.2e}, state {es:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 1e-3


def test_longest_prefill_sequence_matches_oracle(gpu):
    """One sequence at the top of the prefill length range (8192 tokens), two
    heads, against the float64 oracle: the error accumulated over 128 chunks
    of the scan stays within tolerance."""
    x = workloads.packed_inputs([8192], 2, 2, 128, 128, seed=23, h0_std=0.02)
    d = x.to(gpu)
    o, st = gdn.chunk_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, initial_state=d.h0,
                                       output_final_state=True, use_qk_l2norm_in_kernel=True,
                                       cu_seqlens=d.cu_seqlens, lengths=x.lengths)
    torch.cuda.synchronize()
    ro, rs = ref.varlen(ref.chunk_gated_delta_rule, x.q, x.k, x.v, x.g, x.beta, x.cu_seqlens.tolist(),
                        initial_state=x.h0)
    eo, es = rel_err(o, ro), rel_err(st, rs)
    print(f"8192 tokens: out rel err {eo:.2e}, state {es:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 1e-3
