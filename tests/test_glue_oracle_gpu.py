"""Decode-layer glue kernels against the oracle's restatements of the
reference (oracle/glue.py, oracle/gdn.py), GPU.

Where a kernel keeps the reference's rounding points the check is 1 bf16 ulp
per element (fp32 summation order may move the last bit).  Where the
reference rounds more often than the kernel -- the conv update (the wheel
rounds the conv output before the SiLU; the kernel, as the causal-conv1d CUDA
update, rounds once) and RoPE (the reference rotates in bf16 with bf16
cos / sin; the kernel in fp32) -- outputs are held to the bf16 tolerance of
2e-2 relative error and the measured error is printed.  Integer / data
movement (conv window shift, ring slots, positions) is bit-exact.
"""
import math

import pytest
import torch

from oracle import gdn as ogdn
from oracle import glue
from yanchor_amd import independent_memory as im
from yanchor_amd import layers
from yanchor_amd import runtime as rt

from conftest import rel_err

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def rnd(*shape, dev, scale=1.0, seed=0, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(*shape, device=dev, generator=g) * scale).to(dtype)


def ulps(x, ref):
    """Largest |x - ref| in units of ref's bf16 ulp (floored at 2^-16 of max|ref|)."""
    xf, rf = x.float().cpu(), ref.float().cpu()
    ulp = torch.clamp(rf.abs() * 2.0 ** -7, min=rf.abs().max() * 2.0 ** -16)
    return ((xf - rf).abs() / ulp).max().item()


def _gdn_setup(b, dev, seed=0, h=32, d=128):
    cfg = rt.ModelConfig()
    conv_dim, vd = 3 * h * d, h * d
    p = conv_dim + vd + 2 * h
    proj = rnd(b, p, dev=dev, scale=2.0, seed=seed + 1)
    proj[:, -h:] = rnd(b, h, dev=dev, scale=8.0, seed=seed + 5)    # a spread that reaches softplus' identity branch
    conv = rnd(b, 3, conv_dim, dev=dev, seed=seed + 2)
    conv_w = rnd(conv_dim, 4, dev=dev, scale=0.5, seed=seed + 3)
    a_log = torch.log(torch.linspace(1.0, 16.0, h, device=dev))
    dt_bias = torch.linspace(-1.0, 12.0, h, device=dev)
    kw = dict(conv_dim=conv_dim, qk_dim=h * d, hv=h, b_offset=conv_dim + vd, a_offset=conv_dim + vd + h)
    return cfg, proj, conv, conv_w, a_log, dt_bias, kw


def _oracle_prep(proj, conv, conv_w, a_log, dt_bias, kw, conv_update=glue.causal_conv1d_update_cuda):
    """The reference's decode prologue on the host: conv update over the
    [B, C, 3] window (the kernel's window is time-major [B, 3, C]) -- by
    default the CUDA backend's update, else the wheel's torch form -- then
    the fused gates."""
    c, hv = kw["conv_dim"], kw["hv"]
    p, st = proj.cpu(), conv.cpu().transpose(1, 2).contiguous()
    mixed = conv_update(p[:, :c, None], st, conv_w.cpu())[..., 0]
    beta, g = glue.gdn_gates(p[:, kw["b_offset"]: kw["b_offset"] + hv], p[:, kw["a_offset"]: kw["a_offset"] + hv],
                             a_log.cpu(), dt_bias.cpu())
    return mixed, st.transpose(1, 2), beta, g


@pytest.mark.parametrize("b", [1, 5, 128])
def test_gdn_decode_prep_matches_oracle(gpu, b):
    cfg, proj, conv, conv_w, a_log, dt_bias, kw = _gdn_setup(b, gpu)
    conv_before = conv.clone()
    mixed, window, beta, g = _oracle_prep(proj, conv, conv_w, a_log, dt_bias, kw)
    q, k, v, gg, bb = layers.gdn_decode_prep(proj, conv, conv_w, a_log, dt_bias, **kw)
    torch.cuda.synchronize()
    assert torch.equal(conv.cpu(), window)                          # the window shifted by one token
    got = torch.cat((q, k, v), -1).cpu()
    # the CUDA backend's conv update (one rounding): 1 ulp (fp32 sum order)
    assert ulps(got, mixed) <= 1.0001
    # the wheel's torch update rounds the conv output before the SiLU as well
    torch_form = _oracle_prep(proj, conv_before, conv_w, a_log, dt_bias, kw, glue.causal_conv1d_update)[0]
    err = rel_err(got, torch_form)
    print(f"B={b}: conv + SiLU vs the torch form rel err {err:.2e}, max {ulps(got, torch_form):.1f} ulp",
          flush=True)
    assert err <= BF16_TOL
    assert torch.equal(bb.cpu(), beta.float())                      # sigmoid rounded to bf16, as stored
    assert rel_err(gg, g) <= 1e-6


@pytest.mark.parametrize("b", [1, 5, 128])
def test_gdn_decode_fused_matches_oracle(gpu, b):
    """One GDN layer's decode core (conv update, gates, gated delta rule,
    gated RMSNorm) against the reference's CUDA decode path chained on the
    host (_fused_gdn_gate_native_decode_forward, inference_kernels.py:693-721):
    fused gates, the causal-conv1d update, the recurrence in float64 from the
    oracle's bf16 q / k / v, the gated norm."""
    h, d = 32, 128
    cfg, proj, conv, conv_w, a_log, dt_bias, kw = _gdn_setup(b, gpu, seed=20)
    state = rnd(b, h, d, d, dev=gpu, scale=0.02, seed=24, dtype=torch.float32)
    norm_w = (1.0 + rnd(d, dev=gpu, scale=0.1, seed=25).float()).to(torch.bfloat16)
    mixed, _, beta, g = _oracle_prep(proj, conv, conv_w, a_log, dt_bias, kw)
    st0 = state.cpu()
    qk = h * d
    q, k, v = (mixed[:, s:e].reshape(b, 1, h, d) for s, e in ((0, qk), (qk, 2 * qk), (2 * qk, 3 * qk)))
    o, st1 = ogdn.recurrent_gated_delta_rule(q, k, v, g[:, None], beta[:, None].float(), st0)
    z = proj.cpu()[:, kw["conv_dim"]: kw["conv_dim"] + h * d].reshape(b, h, d)
    want = glue.gated_rms_norm(o[:, 0].to(torch.bfloat16), z, norm_w.cpu(), 1e-6).reshape(b, h * d)
    got = layers.gdn_decode_fused(proj, conv, conv_w, a_log, dt_bias, state, norm_w, 1e-6, heads=h, head_dim=d,
                                  z_offset=kw["conv_dim"], b_offset=kw["b_offset"], a_offset=kw["a_offset"])
    torch.cuda.synchronize()
    e_out, e_state = rel_err(got, want), rel_err(state, st1)
    print(f"B={b}: fused GDN core output rel err {e_out:.2e}, state {e_state:.2e}", flush=True)
    assert e_out <= BF16_TOL and e_state <= 1e-3


@pytest.mark.parametrize("b,h", [(1, 32), (128, 32), (3, 5)])
def test_gated_rmsnorm_matches_oracle(gpu, b, h):
    o = rnd(b, h, 128, dev=gpu, scale=0.3, seed=10)
    proj = rnd(b, h * 128 + 96, dev=gpu, seed=11)
    z = proj[:, 32: 32 + h * 128]
    w = (1.0 + rnd(128, dev=gpu, scale=0.1, seed=12).float()).to(torch.bfloat16)
    got = layers.gated_rmsnorm(o, z, w, 1e-6).cpu()
    want = glue.gated_rms_norm(o.cpu(), z.cpu().reshape(b, h, 128), w.cpu(), 1e-6).reshape(b, h * 128)
    # three roundings (normed row, times w, times silu(z)): a 1-ulp flip of
    # the first (fp32 sum order of the norm) carries through the other two
    assert ulps(got, want) <= 2.0001
    assert (got != want).float().mean().item() <= 0.02


@pytest.mark.parametrize("n,d", [(1, 2560), (130, 2560), (7, 256)])
def test_rmsnorm_matches_oracle(gpu, n, d):
    x = rnd(n, d, dev=gpu, scale=3.0, seed=1)
    w = rnd(d, dev=gpu, scale=0.1, seed=3)
    got = layers.rmsnorm(x, w, 1e-6).cpu()
    want = glue.rms_norm(x.cpu(), w.cpu(), 1e-6)
    assert ulps(got, want) <= 1.0001
    assert (got != want).float().mean().item() <= 0.02


def _rope_tables(pos, cfg, dtype):
    return glue.rope_cos_sin(pos.cpu(), rt.rope_inv_freq(cfg, "cpu"), dtype)


@pytest.mark.parametrize("rd", [32, 64, 128])
def test_head_norm_rope_matches_oracle(gpu, rd):
    """q_norm + RoPE: the reference rotates the bf16 normed heads with bf16
    cos / sin tables; the kernel rotates in fp32."""
    n, h = 37, 8
    x = rnd(n, h, 256, dev=gpu, scale=2.0, seed=14)[..., :128]
    w = rnd(128, dev=gpu, scale=0.1, seed=15)
    pos = torch.randint(0, 100000, (n,), device=gpu)
    cfg = rt.ModelConfig(rotary_dim=rd)
    cos, sin = rt.rope_tables(pos, cfg)
    got = layers.head_norm_rope(x, w, cos, sin, rd, 1e-6).cpu()
    c16, s16 = _rope_tables(pos, cfg, torch.bfloat16)
    want = glue.memory_rope(glue.rms_norm(x.cpu(), w.cpu(), 1e-6), c16[:, None], s16[:, None])
    err = rel_err(got, want)
    print(f"rotary {rd}: rel err {err:.2e}", flush=True)
    assert err <= BF16_TOL
    assert torch.equal(got[..., rd:], want[..., rd:]) or ulps(got[..., rd:], want[..., rd:]) <= 1.0001


def test_ring_write_matches_oracle(gpu):
    """k_norm + RoPE of the key heads, then the ring write of key, value and
    position into slot position % window (modeling_yanchor.py:835-843,
    inference_kernels.py:1828-1856)."""
    b, kvh, win, d = 6, 4, 16, 128
    cfg = rt.ModelConfig()
    proj = rnd(b, 2 * kvh * d + 64, dev=gpu, seed=40)
    k = proj[:, :kvh * d].view(b, kvh, d)
    v = proj[:, kvh * d: 2 * kvh * d].view(b, kvh, d)
    w = rnd(d, dev=gpu, scale=0.1, seed=41)
    pos = torch.tensor([0, 5, 15, 16, 33, 1000], device=gpu)
    cos, sin = rt.rope_tables(pos, cfg)
    rows = torch.arange(b, device=gpu) * kvh * win + pos % win
    ring = [rnd(b, kvh, win, d, dev=gpu, seed=42), rnd(b, kvh, win, d, dev=gpu, seed=43),
            torch.full((b, kvh, win), -1, device=gpu, dtype=torch.int32)]
    before = [t.cpu() for t in ring]
    layers.ring_write(k, v, w, cos, sin, rows, pos, *ring, cfg.rotary_dim, 1e-6)
    c16, s16 = _rope_tables(pos, cfg, torch.bfloat16)
    key = glue.memory_rope(glue.rms_norm(k.cpu(), w.cpu(), 1e-6), c16[:, None], s16[:, None])
    rk, rv = before[0].clone(), before[1].clone()
    valid = torch.zeros(b, win, dtype=torch.bool)
    glue.ring_write(rk, rv, valid, key, v.cpu(), torch.ones(b, dtype=torch.bool), (pos % win).cpu())
    got_k, got_v, got_p = (t.cpu() for t in ring)
    assert torch.equal(got_v, rv)
    slot = valid[:, None, :].expand(b, kvh, win)
    assert torch.equal(got_k[~slot], rk[~slot])
    assert rel_err(got_k[slot], rk[slot]) <= BF16_TOL
    want_p = before[2].clone()
    want_p[torch.arange(b), :, (pos % win).cpu()] = pos.cpu().to(torch.int32)[:, None]
    assert torch.equal(got_p, want_p)


@pytest.mark.parametrize("b,g,h,win,live", [(4, 2, 8, 128, 0.8), (128, 8, 32, 1024, 1.0), (3, 1, 4, 64, 0.1)])
def test_window_attend_matches_oracle(gpu, b, g, h, win, live):
    """The SWA physical-ring decode read against the reference's masked
    softmax (inference_kernels.py:1881-1898), with and without the output gate."""
    d = 128
    gen = torch.Generator(device=gpu).manual_seed(80 + b)
    keys = torch.randn(b, g, win, d, device=gpu, generator=gen).to(torch.bfloat16)
    vals = torch.randn(b, g, win, d, device=gpu, generator=gen).to(torch.bfloat16)
    slot_live = torch.rand(b, win, device=gpu, generator=gen) < live
    slot_live[:, 0] = True
    pos = torch.where(slot_live, torch.arange(win, device=gpu, dtype=torch.int32), -1)[:, None].expand(b, g, win)
    pos = pos.contiguous()
    q = torch.randn(b, 1, h, d, device=gpu, generator=gen).to(torch.bfloat16)
    qg = torch.randn(b, h, 2 * d, device=gpu, generator=gen).to(torch.bfloat16)
    gate = qg[..., d:]
    plain = im.ring_decode_attention(q, keys, vals, pos).cpu()
    gated = im.ring_decode_attention(q, keys, vals, pos, gate=gate).cpu()
    valid = slot_live.cpu()
    want = glue.ring_decode_attention(q.cpu(), keys.cpu(), vals.cpu(), valid)
    exact = glue.ring_decode_attention(q.cpu().double(), keys.cpu().double(), vals.cpu().double(), valid)
    want_g = glue.ring_decode_attention(q.cpu(), keys.cpu(), vals.cpu(), valid, gate.cpu())
    e_plain, e_exact, e_gated = rel_err(plain, want), rel_err(plain, exact), rel_err(gated, want_g)
    print(f"B={b} G={g} H={h} W={win}: read {e_plain:.2e} (vs float64 {e_exact:.2e}), gated {e_gated:.2e}",
          flush=True)
    assert e_plain <= BF16_TOL and e_exact <= BF16_TOL and e_gated <= BF16_TOL
    assert ulps(plain, want) <= 2.0001


@pytest.mark.parametrize("g,h", [(8, 32), (2, 4), (4, 4)])
def test_window_attend_dead_blocks(gpu, g, h):
    """Rings that fill from slot 0 (a sequence shorter than the window) and
    rings with whole 16-slot blocks dead between live ones: the read skips
    blocks without a live slot, and must equal the masked softmax over the
    whole ring (inference_kernels.py:1881-1898).  Live counts sit on and beside
    block edges; dead slots hold large garbage so a skipped block that was
    still summed would show."""
    d, win = 128, 1024
    lengths = [1, 2, 15, 16, 17, 31, 32, 33, 64, 100, 500, 1007, 1008, 1023, 1024]
    b = len(lengths) + 3
    gen = torch.Generator(device=gpu).manual_seed(97)
    keys = torch.randn(b, g, win, d, device=gpu, generator=gen).to(torch.bfloat16)
    vals = torch.randn(b, g, win, d, device=gpu, generator=gen).to(torch.bfloat16)
    slot = torch.arange(win, device=gpu)
    live = torch.zeros(b, win, dtype=torch.bool, device=gpu)
    for r, n in enumerate(lengths):
        live[r, :n] = True
    live[len(lengths), (slot // 16) % 3 == 1] = True              # one live block in three
    live[len(lengths) + 1, 1000] = True                           # one live slot, in the last blocks
    live[len(lengths) + 2, (slot // 16) % 2 == 0] = True          # even blocks: one wave's share only
    live[len(lengths) + 2, 16 * 7 + 5] = True                     # and one slot of an odd block
    keys = torch.where(live[:, None, :, None], keys, torch.full_like(keys, 300.0))
    vals = torch.where(live[:, None, :, None], vals, torch.full_like(vals, 1e4))
    pos = torch.where(live, slot.to(torch.int32), -1)[:, None].expand(b, g, win).contiguous()
    q = torch.randn(b, 1, h, d, device=gpu, generator=gen).to(torch.bfloat16)
    got = im.ring_decode_attention(q, keys, vals, pos).cpu()
    want = glue.ring_decode_attention(q.cpu(), keys.cpu(), vals.cpu(), live.cpu())
    err = rel_err(got, want)
    print(f"G={g} H={h} W={win}, {b} fill patterns: read {err:.2e}", flush=True)
    assert err <= BF16_TOL
    assert ulps(got, want) <= 2.0001
    # per row: every fill pattern, not only the batch as a whole
    for r in range(b):
        assert rel_err(got[r], want[r]) <= BF16_TOL, r


@pytest.mark.parametrize("b", [1, 128])
def test_memory_decode_matches_oracle(gpu, b):
    """The anchor-memory projections of one decode token (input norm, the
    fused q / admission / writer projection, memory_prologue with the
    writer's activation, the k / v projection of [u | act] against
    [W_kv | W_kv W_down], k norm + RoPE) against _query_scores and _write_kv
    restated from the same weights in the reference's order (writer down
    projection, residual, then k / v)."""
    cfg = rt.ModelConfig(layers=4)
    m = rt.Model(cfg, batch=b, device=gpu, seed=31)
    L = m.layers[3]
    assert "m_kv@fused" in L                 # the bf16 model takes the fused k / v projection
    gen = torch.Generator(device=gpu).manual_seed(32)
    for name in ("m_q_norm", "m_k_norm", "m_in_norm"):
        L[name].copy_((torch.randn(L[name].shape, device=gpu, generator=gen) * 0.1).to(L[name].dtype))
    L["read_scale"].copy_(torch.randn(cfg.attn_heads, device=gpu, generator=gen))
    L["read_gate_w"].copy_(torch.randn(cfg.attn_heads, cfg.head_dim, device=gpu, generator=gen) * 0.2)
    hidden = rnd(b, cfg.hidden, dev=gpu, seed=33)
    pos = torch.randint(0, 5000, (b,), device=gpu)
    cos, sin = rt.rope_tables(pos, cfg)
    q, gate, key, value, scores = m._memory_decode(L, hidden, cos, sin)
    torch.cuda.synchronize()
    c = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in L.items()}
    u = glue.rms_norm(hidden.cpu(), c["m_in_norm"], cfg.rms_eps)
    c16, s16 = _rope_tables(pos, cfg, torch.bfloat16)
    H, G, D, I = cfg.attn_heads, cfg.kv_heads, cfg.head_dim, cfg.writer_intermediate
    w_q, w_scores, w_gate = glue.query_scores(u, c["m_q"], c["m_q_norm"], c["read_scale"], c["read_gate_w"],
                                              c["read_gate_b"], c["adm_down"], c["adm_up"], c16, s16, H, cfg.rms_eps)
    w_key, w_val = glue.write_kv(u, c["writer_gate_up"][:I], c["writer_gate_up"][I:], c["writer_down"],
                                 c["m_kv"][: G * D], c["m_kv"][G * D:], c["m_k_norm"], c16, s16, G, cfg.rms_eps)
    errs = {"query": rel_err(q, w_q), "gate": rel_err(gate, w_gate), "scores": rel_err(scores, w_scores),
            "key": rel_err(key, w_key), "value": rel_err(value, w_val)}
    print(f"B={b}: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v <= BF16_TOL for v in errs.values()), errs
