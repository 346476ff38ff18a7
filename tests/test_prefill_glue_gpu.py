"""Refill-prefill kernels of packed, ragged prompt pieces (GPU) against the
oracle:

* ``conv_prefill``: the causal conv1d + SiLU over pieces that continue their
  conv windows equals the decode prologue fed one token at a time, bit for
  bit (same fp32 taps, one rounding), and the oracle's prefill form within
  one bf16 ulp; the window left behind is the last three inputs, exactly;
* ``swa_prefill``: sliding-window causal attention (W = 1024, GQA 32 / 8)
  with the ring as left context against the oracle's reference_swa restated
  in float64 (bf16 outputs, bound 2e-2), on fresh pieces of lengths around
  the 16-token tile and the window and on continuations that start before,
  at and past the window; with and without the output gate; and the last
  token of a piece equals the decode read of the ring the piece leaves;
* ``ring_fill``: the ring rows equal the torch formulation's, bit for bit.
"""
import pytest
import torch

from oracle import glue
from yanchor_amd import independent_memory as im
from yanchor_amd import layers
from yanchor_amd import runtime as rt

from conftest import rel_err

pytestmark = pytest.mark.gpu

H, G, D, W = 32, 8, 128, 1024


def _cu(lengths, dev):
    off = [0]
    for n in lengths:
        off.append(off[-1] + n)
    return torch.tensor(off, dtype=torch.int32, device=dev)


@pytest.mark.parametrize("lengths", [[1, 2, 3, 4, 37], [0, 5, 0, 64, 1]], ids=["short", "with_empty"])
def test_conv_prefill_equals_decode_prologue_token_by_token(gpu, lengths):
    g = torch.Generator().manual_seed(1)
    hv, qk, conv = 4, 2 * 128, 2 * 2 * 128 + 4 * 128
    p = conv + 2 * hv
    n = sum(lengths)
    proj = torch.randn(n, p, generator=g).to(torch.bfloat16).to(gpu)
    window = torch.randn(len(lengths), 3, conv, generator=g).to(torch.bfloat16).to(gpu)
    conv_w = (torch.randn(conv, 4, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    a_log = torch.zeros(hv, device=gpu)
    dt_bias = torch.zeros(hv, device=gpu)
    cu = _cu(lengths, gpu)
    win_k = window.clone()
    out = layers.conv_prefill(proj, win_k, conv_w, cu, conv)
    torch.cuda.synchronize()
    off = 0
    for r, length in enumerate(lengths):
        state = window[r: r + 1].clone()
        for t in range(length):
            q, k, v, _, _ = layers.gdn_decode_prep(proj[off + t: off + t + 1], state, conv_w, a_log, dt_bias,
                                                   conv_dim=conv, qk_dim=qk, hv=hv, b_offset=conv, a_offset=conv + hv)
            assert torch.equal(out[off + t], torch.cat((q, k, v), -1)[0]), (r, t)
        assert torch.equal(win_k[r], state[0]), r
        # the oracle's prefill form, float32 taps (another summation order)
        y, new = glue.causal_conv1d_prefill(proj[off: off + length, :conv].cpu(), window[r].cpu(), conv_w.cpu())
        if length:
            assert torch.allclose(out[off: off + length].cpu().float(), y.float(), rtol=2 ** -7, atol=2 ** -7)
        assert torch.equal(win_k[r].cpu(), new)
        off += length


def _ring(rows, starts, gen, dev):
    """Ring rows holding random keys / values at the min(start, W) positions
    before each start (slot = position % W), positions marked, the rest -1."""
    rk = torch.randn(rows, G, W, D, generator=gen).to(torch.bfloat16)
    rv = torch.randn(rows, G, W, D, generator=gen).to(torch.bfloat16)
    rp = torch.full((rows, G, W), -1, dtype=torch.int32)
    for r, s in enumerate(starts):
        pos = torch.arange(max(0, s - W), s)
        rp[r][:, pos % W] = pos.to(torch.int32)[None]
    return rk.to(dev), rv.to(dev), rp.to(dev)


def _oracle_swa(q, k, v, cu, starts, rk, rv, gate):
    """float64 reference_swa per piece over [ring context | piece keys]."""
    out = torch.zeros(q.shape, dtype=torch.float64)
    cu = cu.tolist()
    for r in range(len(cu) - 1):
        s, e = cu[r], cu[r + 1]
        if s == e:
            continue
        nctx = min(starts[r], W - 1)
        pos = torch.arange(starts[r] - nctx, starts[r])
        kc = torch.cat((rk[r][:, pos % W].transpose(0, 1), k[s:e]), 0).double()
        vc = torch.cat((rv[r][:, pos % W].transpose(0, 1), v[s:e]), 0).double()
        out[s:e] = glue.swa_prefill_attention(q[None, s:e].double(), kc[None], vc[None], W, query_start=nctx)[0]
    if gate is not None:
        out = out * torch.sigmoid(gate.double())
    return out


@pytest.mark.parametrize("case", ["fresh", "continued"])
@pytest.mark.parametrize("gated", [False, True], ids=["plain", "gated"])
def test_swa_prefill_matches_oracle(gpu, case, gated):
    gen = torch.Generator().manual_seed(2 if case == "fresh" else 3)
    if case == "fresh":
        lengths = [1, 15, 16, 17, 63, 64, 65, 700, 1500, 2500]
        starts = [0] * len(lengths)
    else:
        lengths = [40, 1, 64, 100, 1030, 0, 17]
        starts = [5, 1023, 1024, 3000, 700, 10, 0]
    n = sum(lengths)
    q = torch.randn(n, H, D, generator=gen).to(torch.bfloat16)
    kv = torch.randn(n, 2 * G, D, generator=gen).to(torch.bfloat16)      # k | v as columns of one row
    gate = torch.randn(n, H, 2 * D, generator=gen).to(torch.bfloat16)[..., D:] if gated else None
    rk, rv, _ = _ring(len(lengths), starts, gen, "cpu")
    cu = _cu(lengths, "cpu")
    qd, kvd = q.to(gpu), kv.to(gpu)
    out = layers.swa_prefill(qd, kvd[:, :G], kvd[:, G:], cu.to(gpu), torch.tensor(starts), rk.to(gpu), rv.to(gpu),
                             torch.arange(len(lengths)), gate=None if gate is None else gate.to(gpu))
    torch.cuda.synchronize()
    want = _oracle_swa(q, kv[:, :G], kv[:, G:], cu, starts, rk, rv, gate)
    err = rel_err(out, want)
    print(f"{case} gated={gated}: rel err {err:.2e} over {n} tokens", flush=True)
    assert err <= 2e-2, err
    # every piece on its own too (no piece leaks into another)
    c = cu.tolist()
    for r in range(len(lengths)):
        if lengths[r]:
            e = rel_err(out[c[r]: c[r + 1]], want[c[r]: c[r + 1]])
            assert e <= 2e-2, (r, e)


def test_ring_fill_and_decode_read_after_prefill(gpu):
    """ring_fill leaves the torch formulation's ring bit for bit, and the
    decode read of a piece's last query over that ring equals the prefill's
    output for it (the same W keys)."""
    gen = torch.Generator().manual_seed(4)
    lengths, starts = [3, 1500, 64, 1100], [0, 0, 1000, 50]
    n = sum(lengths)
    q = torch.randn(n, H, D, generator=gen).to(torch.bfloat16).to(gpu)
    k = torch.randn(n, G, D, generator=gen).to(torch.bfloat16).to(gpu)
    v = torch.randn(n, G, D, generator=gen).to(torch.bfloat16).to(gpu)
    rk, rv, rp = _ring(len(lengths), starts, gen, gpu)
    cu = _cu(lengths, gpu)
    st, rows = torch.tensor(starts), torch.arange(len(lengths))
    out = layers.swa_prefill(q, k, v, cu, st, rk, rv, rows)
    mine = [x.clone() for x in (rk, rv, rp)]
    layers.ring_fill(k, v, cu, st, rows, *mine)
    theirs = [x.clone() for x in (rk, rv, rp)]
    rt.TorchGlue.ring_fill(k, v, cu, st, rows, *theirs, lengths)
    torch.cuda.synchronize()
    for a, b in zip(mine, theirs):
        assert torch.equal(a, b)
    last = (cu[1:] - 1).long()
    read = im.ring_decode_attention(q[last][:, None], mine[0], mine[1], mine[2])
    err = rel_err(read[:, 0], out[last])
    print(f"decode read vs prefill of the last tokens: rel err {err:.2e}", flush=True)
    assert err <= 1e-2, err


def test_prefill_kernels_reject_bad_offsets(gpu):
    """Offsets past the packed tokens and ring rows past the ring are refused
    on the host, before any launch."""
    q = torch.zeros(8, H, D, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(8, G, D, dtype=torch.bfloat16, device=gpu)
    rk = torch.zeros(1, G, W, D, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="cu_seqlens"):
        layers.swa_prefill(q, k, k, torch.tensor([0, 9], dtype=torch.int32), torch.zeros(1), rk, rk,
                           torch.zeros(1))
    with pytest.raises(ValueError, match="ring"):
        layers.swa_prefill(q, k, k, torch.tensor([0, 8], dtype=torch.int32), torch.zeros(1), rk, rk,
                           torch.ones(1))
