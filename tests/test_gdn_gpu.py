"""GPU parity of the token-recurrent gated delta rule (C-ABI path) with the oracle.

Tolerances (Frobenius relative error against the float64 oracle on the same
inputs): state and float32 outputs <= 1e-3, bf16/fp16 outputs <= 2e-2.
"""
import pytest
import torch

from oracle import gdn as ref
from yanchor_amd import gdn, workloads

from conftest import rel_err

pytestmark = pytest.mark.gpu

STATE_TOL = 1e-3
OUT_TOL = {torch.float32: 1e-3, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _run(x, device, **kw):
    d = x.to(device)
    state = d.state.clone()
    o, s = gdn.recurrent_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, initial_state=state,
                                          state_indices=d.state_indices, **kw)
    torch.cuda.synchronize()
    assert s is state  # updated in place, same tensor returned
    return o.cpu(), s.cpu()


def _oracle(x, **kw):
    if x.state_indices is None:
        s0 = x.state[: x.q.shape[0]]
    else:
        s0 = x.state[x.state_indices.long()]
    o, s = ref.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, s0, **kw)
    return o, s


def _check(x, o, s, dtype):
    ro, rs = _oracle(x)
    assert rel_err(o, ro) <= OUT_TOL[dtype], rel_err(o, ro)
    if x.state_indices is None:
        got = s[: x.q.shape[0]]
    else:
        got = s[x.state_indices.long()]
        # rows outside the live set are untouched
        live = torch.zeros(s.shape[0], dtype=torch.bool)
        live[x.state_indices.long()] = True
        assert torch.equal(s[~live], x.state[~live])
    assert rel_err(got, rs) <= STATE_TOL, rel_err(got, rs)


def test_cpu_reference_config_fp32(gpu):
    """B=2, T=256, H=4, dk=dv=64, fp32 inputs, zero initial state."""
    x = workloads.cpu_gdn_config0()
    o, s = _run(x, gpu)
    _check(x, o, s, torch.float32)


def test_decode_config_ragged_slots(gpu):
    """One decode step, 64 live rows of a 96-row slot pool, HV=32, d=128, bf16 q/k/v."""
    x = workloads.decode_gdn_config1(pool_rows=96)
    o, s = _run(x, gpu)
    _check(x, o, s, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kd,vd", [(128, 128), (64, 64), (128, 64), (64, 128)])
def test_shapes_and_dtypes(gpu, dtype, kd, vd):
    x = workloads.gdn_inputs(3, 5, 2, 4, kd, vd, dtype=dtype, seed=kd + vd + 11, state_std=0.05)
    o, s = _run(x, gpu)
    _check(x, o, s, dtype)


def test_negative_state_index_skips_row(gpu):
    x = workloads.gdn_inputs(4, 1, 4, 4, 128, 128, dtype=torch.bfloat16, seed=5, state_std=0.02,
                             pool_rows=6)
    x.state_indices[1] = -1
    d = x.to(gpu)
    state = d.state.clone()
    o, _ = gdn.recurrent_gated_delta_rule(d.q, d.k, d.v, g=d.g, beta=d.beta, initial_state=state,
                                          state_indices=d.state_indices)
    torch.cuda.synchronize()
    assert torch.count_nonzero(o[1]).item() == 0
    keep = [0, 2, 3]
    idx = x.state_indices[keep].long()
    ro, rs = ref.recurrent_gated_delta_rule(x.q[keep], x.k[keep], x.v[keep], x.g[keep], x.beta[keep],
                                            x.state[idx])
    assert rel_err(o.cpu()[keep], ro) <= 2e-2
    assert rel_err(state.cpu()[idx], rs) <= STATE_TOL
    untouched = torch.ones(6, dtype=torch.bool)
    untouched[idx] = False
    assert torch.equal(state.cpu()[untouched], x.state[untouched])


def test_bf16_gates_and_no_l2norm(gpu):
    x = workloads.gdn_inputs(2, 3, 2, 2, 128, 128, dtype=torch.bfloat16, seed=9, state_std=0.02,
                             gate_dtype=torch.bfloat16)
    o, s = _run(x, gpu, use_qk_l2norm_in_kernel=False)
    ro, rs = ref.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, x.state, use_qk_l2norm=False)
    assert rel_err(o, ro) <= 2e-2 and rel_err(s, rs) <= STATE_TOL


def test_state_not_inplace_when_requested(gpu):
    x = workloads.gdn_inputs(2, 1, 2, 2, 64, 64, dtype=torch.float32, seed=21, state_std=0.1).to(gpu)
    before = x.state.clone()
    _, s = gdn.recurrent_gated_delta_rule(x.q, x.k, x.v, g=x.g, beta=x.beta, initial_state=x.state,
                                          inplace=False)
    torch.cuda.synchronize()
    assert torch.equal(x.state, before) and s is not x.state
