"""Fused decode-layer kernels against their torch formulations (GPU).

Each kernel keeps the torch formulation's bf16 rounding points, so outputs
agree to within one bf16 rounding of values that differ only by fp32
summation order: checked as at most 1 bf16 ulp per element, with all but a
small fraction of elements bit-equal.  Pure data movement (the residual sum,
the conv window shift, ring-slot placement) is checked bit-exact.
"""
import pytest
import torch

from yanchor_amd import layers
from yanchor_amd import runtime as rt
from yanchor_amd.runtime import TorchGlue

from conftest import rel_err

pytestmark = pytest.mark.gpu


def ulp_check(x, ref, max_frac=0.02):
    """bf16 x vs bf16 ref: |x - ref| <= 1 ulp of ref everywhere (or below
    2^-16 of the largest |ref|, where a sum cancels and fp32 ordering alone
    decides the low bits), and at most ``max_frac`` of the elements differ."""
    assert x.shape == ref.shape and x.dtype == ref.dtype == torch.bfloat16
    xf, rf = x.float(), ref.float()
    atol = rf.abs().max() * 2.0 ** -16
    ulp = torch.clamp(rf.abs() * 2.0 ** -7, min=atol)
    bad = (xf - rf).abs() > ulp * 1.0001
    assert not bad.any(), f"{int(bad.sum())} elements beyond 1 ulp; first at {bad.nonzero()[0].tolist()}"
    frac = (xf != rf).float().mean().item()
    assert frac <= max_frac, frac


def rnd(*shape, dev, scale=1.0, seed=0, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(*shape, device=dev, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("n,d", [(1, 2560), (130, 2560), (7, 256), (3, 8192)])
def test_rmsnorm(gpu, n, d):
    x, r = rnd(n, d, dev=gpu, scale=3.0, seed=1), rnd(n, d, dev=gpu, seed=2)
    w = rnd(d, dev=gpu, scale=0.1, seed=3)
    ulp_check(layers.rmsnorm(x, w, 1e-6), TorchGlue.rmsnorm(x, w, 1e-6))
    out, s = layers.rmsnorm(x, w, 1e-6, residual=r)
    ref_out, ref_s = TorchGlue.rmsnorm(x, w, 1e-6, r)
    assert torch.equal(s, ref_s)
    ulp_check(out, ref_out)


def test_rmsnorm_strided_rows(gpu):
    base = rnd(9, 3072, dev=gpu, seed=4)
    x = base[:, :2560]                                   # row stride 3072
    w = rnd(2560, dev=gpu, scale=0.1, seed=5)
    ulp_check(layers.rmsnorm(x, w, 1e-6), TorchGlue.rmsnorm(x.contiguous(), w, 1e-6))


def test_rmsnorm_empty_and_bad(gpu):
    w = rnd(256, dev=gpu, seed=6)
    assert layers.rmsnorm(torch.empty(0, 256, device=gpu, dtype=torch.bfloat16), w, 1e-6).shape == (0, 256)
    with pytest.raises(ValueError):
        layers.rmsnorm(torch.zeros(2, 256, device=gpu), w, 1e-6)     # fp32 activations


@pytest.mark.parametrize("b,d", [(128, 2560), (5, 2560), (3, 512)])
def test_decode_inputs(gpu, b, d):
    """Embedding rows and ring rows / live mask exactly; the first norm equal
    to yh_rmsnorm of the same rows; rotary tables as the torch formulation."""
    cfg = rt.ModelConfig()
    v = 1000
    embed = rnd(v, d, dev=gpu, seed=40)
    w = rnd(d, dev=gpu, scale=0.1, seed=41)
    g = torch.Generator(device=gpu).manual_seed(42)
    tokens = torch.randint(0, v, (b,), device=gpu, generator=g)
    tokens[0] = v + 7                                    # outside the vocabulary: a zero row
    positions = torch.randint(0, 1 << 20, (b,), device=gpu, generator=g)
    finished = torch.rand(b, device=gpu, generator=g) < 0.3
    slot_rows = torch.randint(-1, 4, (b,), device=gpu, generator=g)
    inv = rt.rope_inv_freq(cfg, gpu)
    kw = dict(ring_stride=cfg.kv_heads * cfg.swa_window, window=cfg.swa_window)
    h, xn, cos, sin, rows, valid = layers.decode_inputs(tokens, positions, embed, w, inv, 1e-6, finished=finished,
                                                        slot_rows=slot_rows, **kw)
    want_h = embed[tokens.clamp(max=v - 1)].clone()
    want_h[0] = 0
    assert torch.equal(h, want_h)
    assert torch.equal(xn, layers.rmsnorm(want_h, w, 1e-6))
    ulp_check(xn, TorchGlue.rmsnorm(want_h, w, 1e-6))
    rcos, rsin = rt.rope_tables(positions, cfg)
    for got, want in ((cos, rcos), (sin, rsin)):
        assert got.shape == want.shape == (b, cfg.rotary_dim)
        assert (got - want).abs().max().item() <= 2.0 ** -23
    assert torch.equal(rows, torch.arange(b, device=gpu) * kw["ring_stride"] + positions % kw["window"])
    assert torch.equal(valid, (~finished) & (slot_rows >= 0))
    assert layers.decode_inputs(tokens, positions, embed, w, inv, 1e-6, **kw)[5] is None


@pytest.mark.parametrize("b", [1, 5, 128])
def test_gdn_decode_prep(gpu, b):
    cfg = rt.ModelConfig()
    hv, vd = cfg.gdn_heads_v, cfg.gdn_heads_v * cfg.gdn_dv
    p = cfg.conv_dim + vd + 2 * hv
    proj = rnd(b, p, dev=gpu, scale=2.0, seed=7)
    conv = rnd(b, 3, cfg.conv_dim, dev=gpu, seed=8)
    conv_w = rnd(cfg.conv_dim, 4, dev=gpu, scale=0.5, seed=9)
    a_log = torch.log(torch.linspace(1.0, 16.0, hv, device=gpu))
    dt_bias = torch.linspace(-1.0, 1.0, hv, device=gpu)
    kw = dict(conv_dim=cfg.conv_dim, qk_dim=cfg.gdn_heads_k * cfg.gdn_dk, hv=hv, b_offset=cfg.conv_dim + vd,
              a_offset=cfg.conv_dim + vd + hv)
    conv_ref = conv.clone()
    got = layers.gdn_decode_prep(proj, conv, conv_w, a_log, dt_bias, **kw)
    ref = TorchGlue.gdn_prep(proj, conv_ref, conv_w, a_log, dt_bias, **kw)
    assert torch.equal(conv, conv_ref)                   # window shifted by one token
    for x, r in zip(got[:3], ref[:3]):
        ulp_check(x, r.contiguous())
    for x, r in zip(got[3:], ref[3:]):
        assert rel_err(x, r) <= 1e-6


def test_gdn_decode_prep_large_gate_softplus(gpu):
    """a + dt_bias above the softplus threshold (20) takes the identity branch."""
    hv = 4
    proj = torch.zeros(2, 256 * 3 + 2 * hv, device=gpu, dtype=torch.bfloat16)
    proj[:, -hv:] = torch.tensor([25.0, 19.0, -30.0, 0.0])
    conv = torch.zeros(2, 3, 256 * 3, device=gpu, dtype=torch.bfloat16)
    kw = dict(conv_dim=256 * 3, qk_dim=256, hv=hv, b_offset=256 * 3, a_offset=256 * 3 + hv)
    a_log, dt = torch.zeros(hv, device=gpu), torch.zeros(hv, device=gpu)
    got = layers.gdn_decode_prep(proj, conv, torch.ones(768, 4, device=gpu, dtype=torch.bfloat16), a_log, dt, **kw)
    ref = TorchGlue.gdn_prep(proj, conv.clone(), torch.ones(768, 4, device=gpu, dtype=torch.bfloat16), a_log, dt,
                             **kw)
    assert rel_err(got[3], ref[3]) <= 1e-6 and rel_err(got[4], ref[4]) <= 1e-6


@pytest.mark.parametrize("b,h", [(1, 32), (128, 32), (3, 5)])
def test_gated_rmsnorm(gpu, b, h):
    o = rnd(b, h, 128, dev=gpu, scale=0.3, seed=10)
    proj = rnd(b, h * 128 + 96, dev=gpu, seed=11)
    z = proj[:, 32: 32 + h * 128]                         # strided view, as in the projection
    w = (1.0 + rnd(128, dev=gpu, scale=0.1, seed=12).float()).to(torch.bfloat16)
    ulp_check(layers.gated_rmsnorm(o, z, w, 1e-6), TorchGlue.gated_rmsnorm(o, z, w, 1e-6))


@pytest.mark.parametrize("n,i", [(1, 9728), (128, 9728), (5, 2560), (3, 8)])
def test_silu_mul(gpu, n, i):
    gu = rnd(n, 2 * i, dev=gpu, scale=3.0, seed=13)
    ulp_check(layers.silu_mul(gu), TorchGlue.silu_mul(gu))


@pytest.mark.parametrize("rd", [0, 32, 64, 128])
def test_head_norm_rope(gpu, rd):
    n, h = 37, 8
    proj = rnd(n, h, 256, dev=gpu, scale=2.0, seed=14)
    x = proj[..., :128]                                   # head stride 256, as in the fused q | gate layout
    w = rnd(128, dev=gpu, scale=0.1, seed=15)
    pos = torch.randint(0, 100000, (n,), device=gpu)
    cfg = rt.ModelConfig(rotary_dim=max(rd, 2))
    cos, sin = rt.rope_tables(pos, cfg)
    ulp_check(layers.head_norm_rope(x, w, cos, sin, rd, 1e-6),
              TorchGlue.head_norm_rope(x.contiguous(), w, cos, sin, rd, 1e-6))


def test_head_norm_rope_ring_write(gpu):
    """Keys land in ring slot positions % window of each row, nothing else moves."""
    b, kvh, win, d = 6, 4, 16, 128
    x = rnd(b, kvh, d, dev=gpu, seed=16)
    w = rnd(d, dev=gpu, scale=0.1, seed=17)
    pos = torch.tensor([0, 5, 15, 16, 33, 1000], device=gpu)
    cos, sin = rt.rope_tables(pos, rt.ModelConfig())
    ring = rnd(b, kvh, win, d, dev=gpu, seed=18)
    ring_ref = ring.clone()
    rows = torch.arange(b, device=gpu) * kvh * win + pos % win
    kw = dict(out_tok_index=rows, out_tok_stride=d, out_head_stride=win * d)
    layers.head_norm_rope(x, w, cos, sin, 32, 1e-6, out=ring, **kw)
    TorchGlue.head_norm_rope(x, w, cos, sin, 32, 1e-6, out=ring_ref, **kw)
    touched = torch.zeros(b, kvh, win, dtype=torch.bool, device=gpu)
    touched[torch.arange(b, device=gpu), :, pos % win] = True
    assert torch.equal(ring[~touched], ring_ref[~touched])
    ulp_check(ring[touched], ring_ref[touched])


@pytest.mark.parametrize("m,n,k", [(128, 2560, 4096), (128, 12352, 2560), (128, 2560, 9728), (1, 64, 64),
                                   (37, 192, 320), (64, 19456, 2560), (100, 2048, 2560)])
def test_linear_matches_fp32_reference(gpu, m, n, k):
    """fp32-accumulated product rounded once to bf16, as F.linear; the order
    of the fp32 sums differs, so outputs agree to 1 bf16 ulp."""
    x = rnd(m, k, dev=gpu, seed=m + n)
    w = rnd(n, k, dev=gpu, scale=0.02, seed=k)
    ref = (x.float() @ w.float().t()).to(torch.bfloat16)
    got = layers.linear(x, w)
    ulp_check(got, ref, max_frac=0.05)


@pytest.mark.parametrize("split", [1, 2, 5, 16])
def test_linear_split_k_is_deterministic(gpu, split):
    """Every split gives the same result on repeated calls (fixed-order
    partial sums), including after a call with a different shape on the same
    workspace."""
    x = rnd(128, 4096, dev=gpu, seed=1)
    w = rnd(2560, 4096, dev=gpu, scale=0.02, seed=2)
    a = layers.linear(x, w, split_k=split)
    layers.linear(rnd(64, 1024, dev=gpu, seed=3), rnd(640, 1024, dev=gpu, seed=4), split_k=4)
    b = layers.linear(x, w, split_k=split)
    assert torch.equal(a, b)
    ulp_check(a, (x.float() @ w.float().t()).to(torch.bfloat16), max_frac=0.05)


def test_linear_strided_rows(gpu):
    base = rnd(16, 3072, dev=gpu, seed=5)
    x = base[:, 512:]                                    # row stride 3072, 1024-byte offset
    w = rnd(128, 2560, dev=gpu, seed=6)
    ulp_check(layers.linear(x, w), (x.float() @ w.float().t()).to(torch.bfloat16))


@pytest.mark.parametrize("pair", [False, True])
def test_pack_layout(gpu, pair):
    """yh_linear_pack's documented order, bit for bit: K blocks of 32
    outermost, then the N/16 column tiles, then the 64 lanes of a 16x16x32
    MFMA B operand (lane l = 16 q + r holds row 16 T + r, K 32 kb + 8 q ..
    + 8); paired halves interleave the tiles of the two row halves."""
    n, k = 96, 256
    w = rnd(n, k, dev=gpu, seed=5)
    pw = layers.PackedWeight(w, pair_halves=pair)
    src = w.cpu()
    if pair:   # tile 2j = rows 16j.., tile 2j+1 = rows n/2 + 16j..
        src = src.view(2, n // 32, 16, k).permute(1, 0, 2, 3).reshape(n, k)
    want = src.view(n // 16, 16, k // 32, 4, 8).permute(2, 0, 3, 1, 4).reshape(-1)
    torch.cuda.synchronize()
    assert torch.equal(pw.data.cpu(), want)
    with pytest.raises(ValueError):
        layers.PackedWeight(rnd(32, 96, dev=gpu, seed=31))           # K not a multiple of 128


@pytest.mark.parametrize("m,n,k", [(256, 2560, 9728), (256, 10240, 2560), (200, 2576, 2560), (129, 19456, 2560),
                                   (128, 2560, 4096), (128, 19456, 2560), (128, 2560, 9728), (1, 16, 128),
                                   (37, 192, 384), (64, 2048, 2560), (100, 2576, 2560), (17, 4096, 1024)])
def test_linear_packed_matches_fp32_reference(gpu, m, n, k):
    """fp32-accumulated product rounded once to bf16, as F.linear (1 bf16 ulp)."""
    x = rnd(m, k, dev=gpu, seed=m + n + 1)
    w = rnd(n, k, dev=gpu, scale=0.02, seed=k + 1)
    ref = (x.float() @ w.float().t()).to(torch.bfloat16)
    got = layers.linear(x, layers.PackedWeight(w))
    ulp_check(got, ref, max_frac=0.05)


@pytest.mark.parametrize("split", [1, 2, 3, 7, 32])
def test_linear_packed_split_is_deterministic(gpu, split):
    x = rnd(128, 4096, dev=gpu, seed=7)
    pw = layers.PackedWeight(rnd(2560, 4096, dev=gpu, scale=0.02, seed=8))
    a = layers.linear(x, pw, split_k=split)
    layers.linear(rnd(64, 1024, dev=gpu, seed=9), layers.PackedWeight(rnd(640, 1024, dev=gpu, seed=10)), split_k=4)
    b = layers.linear(x, pw, split_k=split)
    assert torch.equal(a, b)
    ulp_check(a, (x.float() @ rnd(2560, 4096, dev=gpu, scale=0.02, seed=8).float().t()).to(torch.bfloat16),
              max_frac=0.05)


def test_linear_packed_strided_rows_and_empty(gpu):
    base = rnd(16, 3072, dev=gpu, seed=11)
    x = base[:, 512:]                                    # row stride 3072, 1024-byte offset
    w = rnd(128, 2560, dev=gpu, seed=12)
    pw = layers.PackedWeight(w)
    ulp_check(layers.linear(x, pw), (x.float() @ w.float().t()).to(torch.bfloat16))
    assert layers.linear(torch.empty(0, 2560, device=gpu, dtype=torch.bfloat16), pw).shape == (0, 128)


def test_ring_write(gpu):
    """Key heads normed + rotated, raw value heads and positions land in ring
    slot positions % window of each row; nothing else moves."""
    b, kvh, win, d = 6, 4, 16, 128
    proj = rnd(b, 2 * kvh * d + 64, dev=gpu, seed=40)
    k = proj[:, :kvh * d].view(b, kvh, d)
    v = proj[:, kvh * d: 2 * kvh * d].view(b, kvh, d)
    w = rnd(d, dev=gpu, scale=0.1, seed=41)
    pos = torch.tensor([0, 5, 15, 16, 33, 1000], device=gpu)
    cos, sin = rt.rope_tables(pos, rt.ModelConfig())
    rows = torch.arange(b, device=gpu) * kvh * win + pos % win
    ring = [rnd(b, kvh, win, d, dev=gpu, seed=42), rnd(b, kvh, win, d, dev=gpu, seed=43),
            torch.randint(-1, 100, (b, kvh, win), device=gpu, dtype=torch.int32)]
    ref = [t.clone() for t in ring]
    layers.ring_write(k, v, w, cos, sin, rows, pos, *ring, 32, 1e-6)
    TorchGlue.ring_write(k, v, w, cos, sin, rows, pos, *ref, 32, 1e-6)
    touched = torch.zeros(b, kvh, win, dtype=torch.bool, device=gpu)
    touched[torch.arange(b, device=gpu), :, pos % win] = True
    assert torch.equal(ring[0][~touched], ref[0][~touched])
    ulp_check(ring[0][touched], ref[0][touched])
    assert torch.equal(ring[1], ref[1]) and torch.equal(ring[2], ref[2])


@pytest.mark.parametrize("b", [1, 128])
def test_memory_prologue(gpu, b):
    """Query (normed, rotated), read gate and admission scores in one launch
    against the torch formulation."""
    cfg = rt.ModelConfig()
    h, d, a = cfg.attn_heads, cfg.head_dim, cfg.admission_rank
    proj = rnd(b, h * d + a + 512, dev=gpu, scale=2.0, seed=50)
    w = rnd(d, dev=gpu, scale=0.1, seed=51)
    pos = torch.randint(0, 5000, (b,), device=gpu)
    cos, sin = rt.rope_tables(pos, cfg)
    g = torch.Generator(device=gpu).manual_seed(52)
    read_scale = torch.randn(h, device=gpu, generator=g)
    gate_w = torch.randn(h, d, device=gpu, generator=g) * 0.2
    gate_b = torch.randn(h, device=gpu, generator=g)
    adm_up = torch.randn(cfg.kv_heads, a, device=gpu, generator=g) * 0.3
    args = (proj, h, h * d, a, w, cos, sin, read_scale, gate_w, gate_b, adm_up, cfg.rotary_dim, 1e-6)
    q, gate, scores = layers.memory_prologue(*args)
    rq, rgate, rscores = TorchGlue.memory_prologue(*args)
    # The normed heads agree to 1 bf16 ulp (fp32 sum order); RoPE mixes each
    # rotary element with its partner, so a 1-ulp input difference moves the
    # output by up to one input ulp even where the rotation cancels.
    qn = TorchGlue.head_norm_rope(proj[:, : h * d].view(b, h, d), w, None, None, 0, 1e-6).float()
    rd = cfg.rotary_dim
    partner = torch.cat((qn[..., rd // 2: rd], qn[..., : rd // 2], torch.zeros_like(qn[..., rd:])), -1)
    bound = rq.float().abs() * 2.0 ** -7 + (qn.abs() + partner.abs()) * 2.0 ** -7
    bound[..., rd:] = rq.float()[..., rd:].abs() * 2.0 ** -7
    assert ((q.float() - rq.float()).abs() <= bound * 1.0001 + 1e-30).all()
    assert (q != rq).float().mean().item() <= 0.02
    assert rel_err(gate, rgate) <= 1e-5 and rel_err(scores, rscores) <= 1e-5
    # the writer's activation in the same launch: silu_mul's output bit for
    # bit, and the other outputs unchanged by it
    wi = 256
    proj2 = rnd(b, h * d + a + 2 * wi, dev=gpu, scale=2.0, seed=53)
    args2 = (proj2,) + args[1:]
    q1, gate1, scores1 = layers.memory_prologue(*args2)
    q2, gate2, scores2, act = layers.memory_prologue(*args2, act_offset=h * d + a, act_width=wi)
    assert torch.equal(act, layers.silu_mul(proj2[:, h * d + a:]))
    assert torch.equal(q1, q2) and torch.equal(gate1, gate2) and torch.equal(scores1, scores2)
    # ... written into given rows (the [u | act] row of the fused memory k/v
    # projection), the columns before them untouched
    row = torch.full((b, 384 + wi), 7.0, dtype=torch.bfloat16, device=gpu)
    _, _, _, act2 = layers.memory_prologue(*args2, act_offset=h * d + a, act_width=wi, act_out=row[:, 384:])
    assert act2.data_ptr() == row[:, 384:].data_ptr() and torch.equal(row[:, 384:], act)
    assert bool((row[:, :384] == 7.0).all())


@pytest.mark.parametrize("split", [1, 4])
def test_linear_packed_residual(gpu, split):
    """out = bf16(x . W^T) + residual, the residual add fused into the store."""
    x = rnd(128, 2560, dev=gpu, seed=60)
    w = rnd(2560, 2560, dev=gpu, scale=0.02, seed=61)
    base = rnd(128, 3072, dev=gpu, seed=62)
    res = base[:, 256: 256 + 2560]                       # strided residual rows
    got = layers.linear(x, layers.PackedWeight(w), split_k=split, residual=res)
    prod = (x.float() @ w.float().t()).to(torch.bfloat16)
    ref = prod + res
    # the bf16 product may differ by 1 ulp (fp32 sum order); where the add
    # cancels that ulp is large next to the sum
    bound = (ref.float().abs() + prod.float().abs()) * 2.0 ** -7
    assert ((got.float() - ref.float()).abs() <= bound * 1.0001 + 1e-30).all()
    assert (got != ref).float().mean().item() <= 0.05


@pytest.mark.parametrize("m,i,k", [(256, 9728, 2560), (130, 256, 384), (128, 9728, 2560), (37, 256, 384),
                                   (1, 32, 128)])
def test_linear_silu_matches_gemm_then_silu_mul(gpu, m, i, k):
    """The MLP activation from the paired packing equals F.linear followed by
    the silu_mul formulation (to 1 bf16 ulp of the products, which the
    activation then carries)."""
    x = rnd(m, k, dev=gpu, seed=m + i)
    w = rnd(2 * i, k, dev=gpu, scale=0.05, seed=k + i)
    got = layers.linear_silu(x, layers.PackedWeight(w, pair_halves=True))
    gu = (x.float() @ w.float().t()).to(torch.bfloat16)
    ref = TorchGlue.silu_mul(gu)
    g, u = gu.float().chunk(2, -1)
    # a 1-ulp change of gate / up moves the activation by about that ulp times
    # the other factor
    bound = ref.float().abs() * 2.0 ** -7 + (u.abs() + g.abs()) * (g.abs() + u.abs()) * 2.0 ** -7
    assert got.shape == ref.shape
    assert ((got.float() - ref.float()).abs() <= bound * 1.0001 + 1e-30).all()
    assert (got != ref).float().mean().item() <= 0.05


@pytest.mark.parametrize("with_res,split,m", [(False, 8, 128), (True, 8, 128), (True, 3, 128), (True, 13, 128),
                                             (False, 32, 128), (True, 12, 256), (False, 5, 200)])
def test_deferred_split_k_into_rmsnorm_is_exact(gpu, with_res, split, m):
    """A projection whose split-K reduce is left to the following RMSNorm
    gives bit for bit what the reduce kernel + RMSNorm give (slice counts on
    both sides of the in-flight plane groups of 4, 8 and 16; 256-row tiles
    past 128 rows)."""
    x = rnd(m, 4096, dev=gpu, seed=90)
    pw = layers.PackedWeight(rnd(2560, 4096, dev=gpu, scale=0.02, seed=91))
    r = rnd(m, 2560, dev=gpu, seed=92) if with_res else None
    h = rnd(m, 2560, dev=gpu, seed=93)
    w = rnd(2560, dev=gpu, scale=0.1, seed=94)
    p = layers.linear(x, pw, split_k=split, residual=r, defer=True)
    assert isinstance(p, layers.Partials) and p.part.shape[0] > 1
    got, got_h = layers.rmsnorm(p, w, 1e-6, residual=h)
    ref, ref_h = layers.rmsnorm(layers.linear(x, pw, split_k=split, residual=r), w, 1e-6, residual=h)
    assert torch.equal(got, ref) and torch.equal(got_h, ref_h)
    assert torch.is_tensor(layers.linear(x, pw, split_k=1, residual=r, defer=True))   # one slice: nothing deferred


@pytest.mark.parametrize("split", [1, 8])
def test_rmsnorm_second_weight(gpu, split):
    """w2: the same residual sum normed with a second weight, equal to a
    separate RMSNorm of that sum (one launch from partials, two otherwise)."""
    x = rnd(128, 4096, dev=gpu, seed=95)
    pw = layers.PackedWeight(rnd(2560, 4096, dev=gpu, scale=0.02, seed=96))
    h = rnd(128, 2560, dev=gpu, seed=97)
    w, w2 = rnd(2560, dev=gpu, scale=0.1, seed=98), rnd(2560, dev=gpu, scale=0.1, seed=99)
    p = layers.linear(x, pw, split_k=split, defer=True)
    got, got_h, got_u = layers.rmsnorm(p, w, 1e-6, residual=h, w2=w2)
    ref, ref_h = layers.rmsnorm(layers.linear(x, pw, split_k=split), w, 1e-6, residual=h)
    assert torch.equal(got, ref) and torch.equal(got_h, ref_h)
    assert torch.equal(got_u, layers.rmsnorm(ref_h, w2, 1e-6))
    ulp_check(got_u, TorchGlue.rmsnorm(ref_h, w2, 1e-6))
    if split > 1:   # the second output as the first columns of wider rows, the same values
        p = layers.linear(x, pw, split_k=split, defer=True)
        _, _, wide_u = layers.rmsnorm(p, w, 1e-6, residual=h, w2=w2, w2_row=2560 + 512)
        assert wide_u.stride(0) == 2560 + 512 and torch.equal(wide_u, got_u)
        # the decode step's [u | act] row: the norm's wide rows in place, any other u copied
        m = rt.Model.__new__(rt.Model)
        m.cfg = rt.ModelConfig(writer_intermediate=512)
        row = m._memory_row(wide_u)
        assert row.shape == (128, 2560 + 512) and row.data_ptr() == wide_u.data_ptr()
        row = m._memory_row(got_u)
        assert row.data_ptr() != got_u.data_ptr() and torch.equal(row[:, :2560], got_u)


@pytest.mark.parametrize("s1,s2", [(12, 12), (3, 13), (8, 2), (16, 16)])
def test_rmsnorm_two_deferred_projections(gpu, s1, s2):
    """A projection's partials with a second projection's partials as its
    residual (the attention layer's memory and attention output projections):
    bit for bit the second reduced on its own (its bf16 store), then the first
    with that as its store residual, then the norms, w2 included.
    reduce_partials equals the projection's own reduce."""
    x1, x2 = rnd(128, 4096, dev=gpu, seed=100), rnd(128, 4096, dev=gpu, seed=101)
    pw1 = layers.PackedWeight(rnd(2560, 4096, dev=gpu, scale=0.02, seed=102))
    pw2 = layers.PackedWeight(rnd(2560, 4096, dev=gpu, scale=0.02, seed=103))
    h = rnd(128, 2560, dev=gpu, seed=104)
    w, w2 = rnd(2560, dev=gpu, scale=0.1, seed=105), rnd(2560, dev=gpu, scale=0.1, seed=106)
    out = layers.linear(x2, pw2, split_k=s2)
    p2 = layers.linear(x2, pw2, split_k=s2, defer=True)
    assert isinstance(p2, layers.Partials)
    p2 = layers.Partials(p2.part.clone(), None)      # one stream, one workspace: keep the planes
    assert torch.equal(layers.reduce_partials(p2), out)
    p1 = layers.linear(x1, pw1, split_k=s1, defer=True)
    got = layers.rmsnorm(layers.Partials(p1.part, p2), w, 1e-6, residual=h, w2=w2)
    torch.cuda.synchronize()
    got = [t.clone() for t in got]
    ref = layers.rmsnorm(layers.linear(x1, pw1, split_k=s1, residual=out, defer=True), w, 1e-6, residual=h, w2=w2)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    with pytest.raises(ValueError):                  # a residual's partials carry no residual of their own
        layers.rmsnorm(layers.Partials(p1.part, layers.Partials(p2.part, out)), w, 1e-6)


@pytest.mark.parametrize("b", [1, 5, 128])
def test_gdn_decode_fused_fp16_state(gpu, b):
    """The float16 state storage of the reference's throughput profile: bit
    for bit the float32 kernel run on the widened state, with its updated
    state rounded to float16 (to nearest even) and the same output row and
    conv window; a row with a negative state index stays untouched."""
    h, d = 32, 128
    conv_dim, vd = 3 * h * d, h * d
    p = conv_dim + vd + 2 * h
    proj = rnd(b, p, dev=gpu, scale=2.0, seed=70)
    conv = rnd(b, 3, conv_dim, dev=gpu, seed=71)
    conv_w = rnd(conv_dim, 4, dev=gpu, scale=0.5, seed=72)
    a_log = torch.log(torch.linspace(1.0, 16.0, h, device=gpu))
    dt_bias = torch.linspace(-1.0, 1.0, h, device=gpu)
    s16 = rnd(b + 2, h, d, d, dev=gpu, scale=0.1, seed=73, dtype=torch.float16)
    s32 = s16.float()
    norm_w = (1.0 + rnd(d, dev=gpu, scale=0.1, seed=74).float()).to(torch.bfloat16)
    idx = torch.arange(b, device=gpu, dtype=torch.int32) + 2
    idx[b // 2] = -1
    kw = dict(heads=h, head_dim=d, z_offset=conv_dim, b_offset=conv_dim + vd, a_offset=conv_dim + vd + h,
              state_indices=idx)
    c16, c32 = conv.clone(), conv.clone()
    before = s16.clone()
    y16 = layers.gdn_decode_fused(proj, c16, conv_w, a_log, dt_bias, s16, norm_w, 1e-6, **kw)
    y32 = layers.gdn_decode_fused(proj, c32, conv_w, a_log, dt_bias, s32, norm_w, 1e-6, **kw)
    assert torch.equal(y16, y32) and torch.equal(c16, c32)
    assert torch.equal(s16, s32.half())
    untouched = [r for r in range(b + 2) if r not in set(idx.tolist())]
    assert torch.equal(s16[untouched], before[untouched])
    assert b == 1 or not torch.equal(s16, before)        # b = 1: its only row has index -1


def test_gdn_decode_fused_fp16_state_range_ends(gpu):
    """The float16 store at both ends of the range, as torch's float32 ->
    float16 conversion rounds: rows 0-1 hold subnormal states (below 2^-14)
    with tiny values, so the update stays subnormal; rows 2-4 hold states
    near 65504 with a decay of ~1, so the update overflows to inf."""
    b, h, d = 5, 32, 128
    conv_dim, vd = 3 * h * d, h * d
    p = conv_dim + vd + 2 * h
    proj = rnd(b, p, dev=gpu, scale=2.0, seed=80).float()
    conv = rnd(b, 3, conv_dim, dev=gpu, seed=81).float()
    proj[:2, 2 * vd:conv_dim] *= 1e-6                    # v of the tiny rows
    conv[:2, :, 2 * vd:] *= 1e-6
    proj[2:, conv_dim + vd + h:] = -30.0                 # a: softplus ~ 0, decay ~ 1
    proj, conv = proj.to(torch.bfloat16), conv.to(torch.bfloat16)
    conv_w = rnd(conv_dim, 4, dev=gpu, scale=0.5, seed=82)
    a_log = torch.log(torch.linspace(1.0, 16.0, h, device=gpu))
    dt_bias = torch.linspace(-1.0, 1.0, h, device=gpu)
    g = torch.Generator(device=gpu).manual_seed(83)
    sign = torch.where(torch.rand(b, h, d, d, device=gpu, generator=g) < 0.5, -1.0, 1.0)
    tiny = 2.0 ** (-24 + 10 * torch.rand(b, h, d, d, device=gpu, generator=g))      # 2^-24 .. 2^-14
    huge = 60000.0 + 5504.0 * torch.rand(b, h, d, d, device=gpu, generator=g)
    s16 = (sign * torch.where(torch.arange(b, device=gpu)[:, None, None, None] < 2, tiny, huge)).half()
    s32 = s16.float()
    norm_w = (1.0 + rnd(d, dev=gpu, scale=0.1, seed=84).float()).to(torch.bfloat16)
    kw = dict(heads=h, head_dim=d, z_offset=conv_dim, b_offset=conv_dim + vd, a_offset=conv_dim + vd + h)
    c16, c32 = conv.clone(), conv.clone()
    y16 = layers.gdn_decode_fused(proj, c16, conv_w, a_log, dt_bias, s16, norm_w, 1e-6, **kw)
    y32 = layers.gdn_decode_fused(proj, c32, conv_w, a_log, dt_bias, s32, norm_w, 1e-6, **kw)
    assert torch.equal(y16, y32) and torch.equal(c16, c32)
    assert torch.equal(s16, s32.half())
    lo = s16[:2].float().abs()
    assert ((lo > 0) & (lo < 2.0 ** -14)).float().mean() > 0.5   # the subnormal range is exercised
    assert torch.isinf(s16[2:]).any() and torch.isfinite(s16[2:]).any()


@pytest.mark.parametrize("b", [1, 5, 128])
def test_gdn_decode_fused_equals_three_launches(gpu, b, monkeypatch):
    """Conv update + gated delta rule + gated norm in one launch give bit for
    bit what gdn_decode_prep, the recurrence (at its 128-column tile) and
    gated_rmsnorm give: output row, shifted conv window and state; a row with
    a negative state index leaves its state alone."""
    from yanchor_amd import gdn
    monkeypatch.setenv("YH_GDN_TILE", "128:512")
    h, d = 32, 128
    conv_dim, vd = 3 * h * d, h * d
    p = conv_dim + vd + 2 * h
    proj = rnd(b, p + 8, dev=gpu, scale=2.0, seed=60)[:, :p]          # row stride P + 8
    conv = rnd(b, 3, conv_dim, dev=gpu, seed=61)
    conv_w = rnd(conv_dim, 4, dev=gpu, scale=0.5, seed=62)
    a_log = torch.log(torch.linspace(1.0, 16.0, h, device=gpu))
    dt_bias = torch.linspace(-1.0, 1.0, h, device=gpu)
    state = rnd(b + 2, h, d, d, dev=gpu, scale=0.1, seed=63, dtype=torch.float32)
    norm_w = (1.0 + rnd(d, dev=gpu, scale=0.1, seed=64).float()).to(torch.bfloat16)
    idx = torch.arange(b, device=gpu, dtype=torch.int32) + 2
    idx[b // 2] = -1
    kw = dict(conv_dim=conv_dim, qk_dim=h * d, hv=h, b_offset=conv_dim + vd, a_offset=conv_dim + vd + h)
    conv_ref, state_ref = conv.clone(), state.clone()
    q, k, v, g, beta = layers.gdn_decode_prep(proj, conv_ref, conv_w, a_log, dt_bias, **kw)
    o, _ = gdn.recurrent_gated_delta_rule(q.view(b, 1, h, d), k.view(b, 1, h, d), v.view(b, 1, h, d),
                                          g=g.view(b, 1, h), beta=beta.view(b, 1, h), initial_state=state_ref,
                                          use_qk_l2norm_in_kernel=True, state_indices=idx)
    want = layers.gated_rmsnorm(o.view(b, h, d), proj[:, conv_dim: conv_dim + vd], norm_w, 1e-6)
    got = layers.gdn_decode_fused(proj, conv, conv_w, a_log, dt_bias, state, norm_w, 1e-6, heads=h, head_dim=d,
                                  z_offset=conv_dim, b_offset=conv_dim + vd, a_offset=conv_dim + vd + h,
                                  state_indices=idx)
    assert torch.equal(conv, conv_ref)
    assert torch.equal(state, state_ref)
    assert torch.equal(got, want.view(b, h * d))
