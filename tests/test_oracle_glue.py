"""Pins of oracle/glue.py (CPU): each restatement against a library routine
or a closed form, with a planted mistake that must fail where the check
would otherwise be weak."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import glue

from conftest import rel_err


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_rms_norm_matches_torch_rms_norm():
    x = torch.randn(7, 256, generator=_g(1), dtype=torch.float64) * 3
    w = torch.randn(256, generator=_g(2), dtype=torch.float64) * 0.1
    want = F.rms_norm(x, (256,), weight=1.0 + w, eps=1e-6)
    assert rel_err(glue.rms_norm(x, w, 1e-6), want) < 1e-14
    # bf16: one rounding of the fp32 result
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    want_b = F.rms_norm(xb.float(), (256,), weight=1.0 + wb.float(), eps=1e-6).to(torch.bfloat16)
    got_b = glue.rms_norm(xb, wb, 1e-6)
    assert got_b.dtype == torch.bfloat16
    assert ((got_b.float() - want_b.float()).abs() <= want_b.float().abs() * 2 ** -8 + 1e-30).all()


def test_gated_rms_norm_matches_norm_times_silu():
    x = torch.randn(5, 4, 128, generator=_g(3), dtype=torch.float64)
    z = torch.randn(5, 4, 128, generator=_g(4), dtype=torch.float64) * 2
    w = 1 + torch.randn(128, generator=_g(5), dtype=torch.float64) * 0.1
    want = F.rms_norm(x, (128,), weight=w, eps=1e-6) * F.silu(z)
    assert rel_err(glue.gated_rms_norm(x, z, w, 1e-6), want) < 1e-14
    # planted mistake: gating before the norm is a different function
    wrong = F.rms_norm(x * F.silu(z), (128,), weight=w, eps=1e-6)
    assert rel_err(wrong, want) > 0.1


def test_causal_conv1d_update_token_by_token_equals_causal_conv():
    """Feeding a sequence one token at a time through the update (from a zero
    state) equals F.conv1d over the whole causal sequence, in float64; the
    state ends as the last S inputs."""
    b, c, t, k = 2, 12, 9, 4
    x = torch.randn(b, c, t, generator=_g(6), dtype=torch.float64)
    w = torch.randn(c, k, generator=_g(7), dtype=torch.float64)
    state = torch.zeros(b, c, k - 1, dtype=torch.float64)
    outs = [glue.causal_conv1d_update(x[:, :, i:i + 1], state, w) for i in range(t)]
    want = F.silu(F.conv1d(F.pad(x, (k - 1, 0)), w[:, None, :], groups=c))
    assert rel_err(torch.cat(outs, -1), want) < 1e-14
    assert torch.equal(state, x[:, :, -(k - 1):])
    # a wider state (the reference keeps K inputs) gives the same outputs
    state4 = torch.zeros(b, c, k, dtype=torch.float64)
    outs4 = [glue.causal_conv1d_update(x[:, :, i:i + 1], state4, w) for i in range(t)]
    assert rel_err(torch.cat(outs4, -1), want) < 1e-14
    # planted mistake: taps in reverse order
    state = torch.zeros(b, c, k - 1, dtype=torch.float64)
    flipped = [glue.causal_conv1d_update(x[:, :, i:i + 1], state, w.flip(-1)) for i in range(t)]
    assert rel_err(torch.cat(flipped, -1), want) > 0.1


def test_causal_conv1d_update_bf16_rounding_points():
    """In bf16 the conv output is a bf16 tensor (torch's bf16 F.conv1d) and
    the SiLU is applied to that tensor: within one bf16 rounding of each."""
    b, c, k = 3, 64, 4
    x = torch.randn(b, c, 1, generator=_g(8)).to(torch.bfloat16)
    state = torch.randn(b, c, k - 1, generator=_g(9)).to(torch.bfloat16)
    w = (torch.randn(c, k, generator=_g(10)) * 0.5).to(torch.bfloat16)
    full = torch.cat([state, x], -1)
    conv = F.conv1d(full, w[:, None, :], groups=c)                    # bf16 output
    want = F.silu(conv)
    got = glue.causal_conv1d_update(x, state.clone(), w)
    assert got.dtype == torch.bfloat16
    assert ((got.float() - want.float()).abs() <= want.float().abs() * 2 ** -7 + 2 ** -14).all()


def test_cuda_conv_update_equals_torch_form_in_float64_and_rounds_once():
    b, c, k = 3, 64, 4
    x = torch.randn(b, c, 1, generator=_g(30), dtype=torch.float64)
    st = torch.randn(b, c, k - 1, generator=_g(31), dtype=torch.float64)
    w = torch.randn(c, k, generator=_g(32), dtype=torch.float64) * 0.5
    st1, st2 = st.clone(), st.clone()
    assert rel_err(glue.causal_conv1d_update_cuda(x, st1, w), glue.causal_conv1d_update(x, st2, w)) < 1e-15
    assert torch.equal(st1, st2)
    # bf16: one rounding of the fp32 silu(sum) -- within half a bf16 ulp of
    # the float64 result; the torch form's extra rounding of the conv output
    # moves it by at most |silu'| times half an ulp of that output
    xb, sb, wb = x.to(torch.bfloat16), st.to(torch.bfloat16), w.to(torch.bfloat16)
    exact = F.silu((torch.cat([sb, xb], -1).double() * wb.double()[None]).sum(-1, keepdim=True))
    once = glue.causal_conv1d_update_cuda(xb, sb.clone(), wb)
    assert ((once.double() - exact).abs() <= exact.abs() * 2.0 ** -8 + 1e-30).all()
    twice = glue.causal_conv1d_update(xb, sb.clone(), wb)
    pre = (torch.cat([sb, xb], -1).double() * wb.double()[None]).sum(-1, keepdim=True)
    bound = exact.abs() * 2.0 ** -8 + 1.1 * pre.abs() * 2.0 ** -8 + 1e-30
    assert ((twice.double() - exact).abs() <= bound).all()
    assert (once != twice).any()                                      # the two forms are not the same rounding


def test_gdn_gates_against_library_and_closed_form():
    hv = 8
    b = torch.randn(3, hv, generator=_g(11)).to(torch.bfloat16)
    a = (torch.randn(3, hv, generator=_g(12)) * 10).to(torch.bfloat16)
    a[0, 0], a[0, 1] = 25.0, -30.0                               # both softplus branches
    a_log = torch.log(torch.linspace(1, 16, hv))
    dt = torch.linspace(-1, 1, hv)
    beta, g = glue.gdn_gates(b, a, a_log, dt)
    assert beta.dtype == torch.bfloat16 and g.dtype == torch.float32
    assert torch.equal(beta, torch.sigmoid(b.float()).to(torch.bfloat16))
    want_g = -torch.exp(a_log) * F.softplus(a.float() + dt, beta=1.0, threshold=20.0)
    assert rel_err(g, want_g) < 1e-6
    # closed form at a = 0, dt_bias = 0: g = -exp(A_log) * log 2
    _, g0 = glue.gdn_gates(b, torch.zeros_like(a), a_log, torch.zeros(hv))
    assert torch.allclose(g0, -torch.exp(a_log) * math.log(2.0), rtol=1e-6)


def test_memory_rope_is_a_complex_rotation():
    d, rd = 128, 32
    x = torch.randn(4, 3, d, generator=_g(13), dtype=torch.float64)
    pos = torch.tensor([0, 1, 77, 5000])
    inv = 1.0 / (1e7 ** (torch.arange(0, rd // 2, dtype=torch.float64) / (rd // 2)))
    ang = pos[:, None].double() * inv
    cos, sin = torch.cat((ang, ang), -1).cos(), torch.cat((ang, ang), -1).sin()
    got = glue.memory_rope(x, cos[:, None], sin[:, None])
    # (x1 + i x2) e^{i theta} on the rotary pairs (j, j + rd/2)
    z = torch.complex(x[..., : rd // 2], x[..., rd // 2: rd]) * torch.exp(1j * ang)[:, None]
    assert rel_err(got[..., : rd // 2], z.real) < 1e-14 and rel_err(got[..., rd // 2: rd], z.imag) < 1e-14
    assert torch.equal(got[..., rd:], x[..., rd:])
    assert torch.equal(got[0], x[0])                                  # position 0: identity
    # planted mistake: rotating the other way is a different function
    wrong = glue.memory_rope(x, cos[:, None], -sin[:, None])
    assert rel_err(wrong[1:], got[1:]) > 1e-3


def test_read_gate_closed_forms():
    h, d = 6, 128
    q = torch.randn(5, h, d, generator=_g(14), dtype=torch.float64)
    w = torch.randn(h, d, generator=_g(15), dtype=torch.float64)
    bias = torch.randn(h, generator=_g(16), dtype=torch.float64)
    assert torch.equal(glue.query_read_gate(q, torch.zeros(h, dtype=torch.float64), w, bias),
                       torch.zeros(5, h, dtype=torch.float64))
    rs = torch.randn(h, generator=_g(17), dtype=torch.float64)
    gate = glue.query_read_gate(q, rs, w, bias)
    want = torch.tanh(rs) * 2 / (1 + torch.exp(-((q * w).sum(-1) / math.sqrt(d) + bias)))
    assert rel_err(gate, want) < 1e-14
    assert (gate.abs() <= 2 * rs.tanh().abs() + 1e-15).all()


def test_query_scores_and_write_kv_reduce_at_their_initialisation():
    """Position 0 (no rotation) and the reference's zero-initialised writer
    down projection (modeling_yanchor.py:142-144): key = k_norm(k_proj u)."""
    hid, h, g, d, rank, inter = 64, 4, 2, 128, 8, 32
    gen = _g(18)
    dt = torch.float64
    u = torch.randn(3, hid, generator=gen, dtype=dt)
    qp, kp, vp = (torch.randn(n * d, hid, generator=gen, dtype=dt) * 0.1 for n in (h, g, g))
    wg, wu = (torch.randn(inter, hid, generator=gen, dtype=dt) * 0.1 for _ in range(2))
    down = torch.zeros(hid, inter, dtype=dt)
    adm_d, adm_u = torch.randn(rank, hid, generator=gen, dtype=dt), torch.randn(g, rank, generator=gen, dtype=dt)
    qn, kn = (torch.randn(d, generator=gen, dtype=dt) * 0.1 for _ in range(2))
    cos, sin = glue.rope_cos_sin(torch.zeros(3, dtype=torch.long), torch.ones(16), dt)
    key, value = glue.write_kv(u, wg, wu, down, kp, vp, kn, cos, sin, g)
    assert rel_err(key, F.rms_norm((u @ kp.t()).view(3, g, d), (d,), weight=1 + kn, eps=1e-6)) < 1e-14
    assert rel_err(value, (u @ vp.t()).view(3, g, d)) < 1e-14
    q, scores, gate = glue.query_scores(u, qp, qn, torch.zeros(h, dtype=dt), torch.zeros(h, d, dtype=dt),
                                        torch.zeros(h, dtype=dt), adm_d, adm_u, cos, sin, h)
    assert rel_err(q, F.rms_norm((u @ qp.t()).view(3, h, d), (d,), weight=1 + qn, eps=1e-6)) < 1e-14
    assert torch.equal(gate, torch.zeros(3, h, dtype=dt))
    assert scores.dtype == torch.float32
    assert rel_err(scores, F.silu(u @ adm_d.t()) @ adm_u.t()) < 1e-6


def _sdpa_ring(q, k, v, valid):
    """The reference's own call (inference_kernels.py:637) in float64."""
    out = F.scaled_dot_product_attention(q.transpose(1, 2), k, v, attn_mask=valid[:, None, None, :],
                                         dropout_p=0.0, is_causal=False, enable_gqa=q.shape[2] != k.shape[1])
    return out.transpose(1, 2)


def test_ring_decode_attention_matches_sdpa():
    b, g, w, d, h = 3, 2, 48, 128, 8
    gen = _g(19)
    q = torch.randn(b, 1, h, d, generator=gen, dtype=torch.float64)
    k = torch.randn(b, g, w, d, generator=gen, dtype=torch.float64)
    v = torch.randn(b, g, w, d, generator=gen, dtype=torch.float64)
    valid = torch.rand(b, w, generator=gen) < 0.6
    valid[:, 0] = True
    assert rel_err(glue.ring_decode_attention(q, k, v, valid), _sdpa_ring(q, k, v, valid)) < 1e-13
    # planted mistake: query head h on KV head h % G instead of h // (H / G)
    perm = torch.arange(h).view(h // g, g).t().reshape(-1)
    wrong = glue.ring_decode_attention(q[:, :, perm], k, v, valid)[:, :, torch.argsort(perm)]
    assert rel_err(wrong, _sdpa_ring(q, k, v, valid)) > 0.05


def test_ring_decode_attention_closed_forms():
    b, g, w, d, h = 2, 1, 16, 128, 2
    gen = _g(20)
    q = torch.randn(b, 1, h, d, generator=gen, dtype=torch.float64)
    k = torch.randn(b, g, w, d, generator=gen, dtype=torch.float64)
    v = torch.randn(b, g, w, d, generator=gen, dtype=torch.float64)
    one = torch.zeros(b, w, dtype=torch.bool)
    one[:, 5] = True                                                  # one live slot: its value row
    out = glue.ring_decode_attention(q, k, v, one)
    assert rel_err(out, v[:, :, 5][:, :, None].expand(b, g, h, d).reshape(b, 1, h, d)) < 1e-15
    same_k = k[:, :, :1].expand(b, g, w, d)                           # equal keys: mean of the live values
    live = torch.rand(b, w, generator=gen) < 0.5
    live[:, 0] = True
    out = glue.ring_decode_attention(q, same_k, v, live)
    mean = (v * live[:, None, :, None]).sum(2) / live.sum(-1)[:, None, None]
    assert rel_err(out, mean[:, :, None].expand(b, g, h, d).reshape(b, 1, h, d)) < 1e-13
    assert torch.equal(glue.ring_decode_attention(q, k, v, torch.zeros(b, w, dtype=torch.bool)),
                       torch.zeros_like(q))


def test_ring_decode_attention_gate_rounding():
    """bf16: the read is rounded, sigmoid(gate) is rounded, then the product
    (inference_kernels.py:1899-1906)."""
    b, g, w, d, h = 2, 2, 32, 128, 4
    gen = _g(21)
    q = torch.randn(b, 1, h, d, generator=gen).to(torch.bfloat16)
    k, v = (torch.randn(b, g, w, d, generator=gen).to(torch.bfloat16) for _ in range(2))
    valid = torch.ones(b, w, dtype=torch.bool)
    gate = torch.randn(b, h, d, generator=gen).to(torch.bfloat16)
    plain = glue.ring_decode_attention(q, k, v, valid)
    got = glue.ring_decode_attention(q, k, v, valid, gate)
    assert torch.equal(got, plain * torch.sigmoid(gate.float()).to(torch.bfloat16)[:, None])


def test_ring_write_places_one_token():
    b, g, w, d = 3, 2, 8, 4
    rk, rv = torch.zeros(b, g, w, d), torch.zeros(b, g, w, d)
    valid = torch.zeros(b, w, dtype=torch.bool)
    key, val = torch.randn(b, g, d, generator=_g(22)), torch.randn(b, g, d, generator=_g(23))
    glue.ring_write(rk, rv, valid, key, val, torch.tensor([True, False, True]), torch.tensor([0, 3, 7]))
    for i, s in enumerate((0, 3, 7)):
        assert torch.equal(rk[i, :, s], key[i]) and torch.equal(rv[i, :, s], val[i])
    assert valid.sum() == 2 and valid[0, 0] and valid[2, 7] and not valid[1].any()
    assert int((rk != 0).any(-1).sum()) == b * g                   # nothing else written


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_cos_sin_tables(dtype):
    pos = torch.tensor([0, 3, 1000])
    inv = 1.0 / (1e7 ** (torch.arange(0, 16, dtype=torch.float32) / 16))
    cos, sin = glue.rope_cos_sin(pos, inv, dtype)
    assert cos.dtype == dtype and cos.shape == (3, 32)
    assert torch.equal(cos[0], torch.ones(32, dtype=dtype)) and torch.equal(sin[0], torch.zeros(32, dtype=dtype))
    ang = pos[:, None].float() * inv
    assert torch.allclose(cos[:, :16].float(), ang.cos(), atol=1e-2 if dtype == torch.bfloat16 else 1e-6)


def _conv_inputs(t, c, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, c, generator=g, dtype=torch.float64).to(dtype)
    win = torch.randn(3, c, generator=g, dtype=torch.float64).to(dtype)
    w = (torch.randn(c, 4, generator=g, dtype=torch.float64) * 0.5).to(dtype)
    return x, win, w


@pytest.mark.parametrize("dtype", [torch.float64, torch.bfloat16])
@pytest.mark.parametrize("t", [0, 1, 2, 3, 7, 40])
def test_conv_prefill_equals_token_by_token_cuda_update(dtype, t):
    """A piece of t tokens continuing a window reads and leaves what t decode
    updates of the CUDA form (fed one token at a time) read and leave, in
    float64 and in bf16 (both round once per output; within one bf16 ulp)."""
    x, win, w = _conv_inputs(t, 24, dtype, 5 + t)
    y, new_win = glue.causal_conv1d_prefill(x, win, w)
    state = win.t().contiguous()[None].clone()                  # [1, C, 3] oldest first
    outs = [glue.causal_conv1d_update_cuda(x[i][None, :, None], state, w)[0, :, 0] for i in range(t)]
    want = torch.stack(outs) if outs else y
    # the two sum the same four fp32 (float64) products in different orders
    tol = 1e-12 if dtype == torch.float64 else 2.0 ** -7
    assert torch.allclose(y.double(), want.double(), rtol=tol, atol=tol)
    assert torch.equal(new_win, state[0].t())


def test_conv_prefill_from_a_zero_window_is_the_causal_conv():
    """From a zero window in float64: F.conv1d over the causally padded
    sequence, then SiLU; reversed taps (a planted mistake) differ."""
    x, _, w = _conv_inputs(33, 16, torch.float64, 9)
    zero = torch.zeros(3, 16, dtype=torch.float64)
    y, _ = glue.causal_conv1d_prefill(x, zero, w)
    ref = F.silu(F.conv1d(F.pad(x.t()[None], (3, 0)), w[:, None, :], groups=16))[0].t()
    assert torch.allclose(y, ref, rtol=0, atol=1e-12)
    planted, _ = glue.causal_conv1d_prefill(x, zero, w.flip(-1))
    assert not torch.allclose(planted, ref, atol=1e-3)


def _swa_inputs(b, l, h, g, d, seed, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, l, h, d, generator=gen, dtype=torch.float64).to(dtype)
    k = torch.randn(b, l, g, d, generator=gen, dtype=torch.float64).to(dtype)
    v = torch.randn(b, l, g, d, generator=gen, dtype=torch.float64).to(dtype)
    return q, k, v


def test_swa_prefill_inside_the_window_is_causal_sdpa():
    """Window >= length: plain causal attention, F.scaled_dot_product_attention
    with is_causal and enable_gqa (the library routine)."""
    q, k, v = _swa_inputs(2, 37, 8, 2, 16, 1)
    out = glue.swa_prefill_attention(q, k, v, 64)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True,
                                         enable_gqa=True).transpose(1, 2)
    assert torch.allclose(out, ref, atol=1e-12)


def test_swa_prefill_equals_token_by_token_ring_reads():
    """Past the window: every query's output is the decode read of a ring of
    `window` slots after the chronological write of the tokens up to it (the
    decode path's physical ring), so prefill and decode attend alike."""
    b, l, h, g, d, w = 2, 45, 4, 2, 16, 8
    q, k, v = _swa_inputs(b, l, h, g, d, 2)
    out = glue.swa_prefill_attention(q, k, v, w)
    ring_k = torch.zeros(b, g, w, d, dtype=torch.float64)
    ring_v = torch.zeros_like(ring_k)
    valid = torch.zeros(b, w, dtype=torch.bool)
    for t in range(l):
        glue.ring_write(ring_k, ring_v, valid, k[:, t], v[:, t], torch.ones(b, dtype=torch.bool), t % w)
        read = glue.ring_decode_attention(q[:, t:t + 1], ring_k, ring_v, valid)
        assert torch.allclose(out[:, t:t + 1], read, atol=1e-12), t
    # a window one slot too wide (a planted mistake) differs past the window
    wide = glue.swa_prefill_attention(q, k, v, w + 1)
    assert not torch.allclose(wide[:, w:], out[:, w:], atol=1e-6)


def test_swa_prefill_window_one_and_continuation():
    """window = 1: each query returns its own (GQA-shared) value.  A piece
    starting at query_start over all keys equals the tail of the whole
    prefill (the continuation form the chunked prefill uses)."""
    q, k, v = _swa_inputs(1, 20, 4, 2, 8, 3)
    one = glue.swa_prefill_attention(q, k, v, 1)
    assert torch.allclose(one, v.repeat_interleave(2, dim=2), atol=1e-12)
    full = glue.swa_prefill_attention(q, k, v, 6)
    tail = glue.swa_prefill_attention(q[:, 13:], k, v, 6, query_start=13)
    assert torch.allclose(tail, full[:, 13:], atol=1e-12)
