"""The host model ops (oracle/model_ops.py) that the full-model GPU check and
the CPU baseline run: on a small model, one float32 decode step through
``HostOps`` equals the same step through the runtime's torch formulations of
the glue (the definitions the fused kernels are tested against) to float32
rounding, caches included -- so the adapters (the conv window's layout, the
gates, RoPE widths, ring slots, the memory's query side) are wired as the
runtime expects.  The GDN recurrence, the anchor memory and the ring read are
the oracle's in both runs."""
import torch

from oracle.model_ops import HostOps
from yanchor_amd import runtime as rt

from conftest import rel_err


class TorchGlueOps(HostOps):
    """HostOps with the layer glue swapped for the runtime's torch forms."""


for _name in ("decode_inputs", "rmsnorm", "gdn_prep", "gated_rmsnorm", "silu_mul", "head_norm_rope", "ring_write",
              "memory_prologue"):
    setattr(TorchGlueOps, _name, staticmethod(getattr(rt.TorchGlue, _name)))


def _small():
    return rt.ModelConfig(layers=8, hidden=256, intermediate=512, vocab=1000, gdn_heads_k=2, gdn_heads_v=2,
                          attn_heads=4, kv_heads=2, swa_window=64, memory_capacity=32, memory_chunk=8,
                          writer_intermediate=256, admission_rank=16)


def _fill_caches(m, seed):
    g = torch.Generator().manual_seed(seed)
    for t in m.cache_tensors():
        if t.dtype == torch.float32:
            t.copy_(torch.randn(t.shape, generator=g) * 0.1)
    for i in m.ring_pos:
        live = torch.rand(m.ring_pos[i].shape, generator=g) < 0.7
        m.ring_pos[i].copy_(torch.where(live, torch.arange(m.ring_pos[i].shape[-1], dtype=torch.int32), -1))
        st = m.memory[i]
        st.positions.copy_(torch.where(torch.rand(st.positions.shape, generator=g) < 0.8,
                                       torch.arange(st.positions.shape[-1], dtype=torch.int32), -1))
        st.scores.copy_(torch.where(st.positions >= 0, st.scores, torch.full_like(st.scores, -float("inf"))))
        st.count.fill_(3)
        st.total.fill_(40)


def test_host_ops_match_the_runtime_torch_glue():
    cfg = _small()
    b = 5
    models = []
    for ops in (HostOps(), TorchGlueOps()):
        m = rt.Model(cfg, batch=b, device="cpu", seed=3, ops=ops, dtype=torch.float32)
        for L in m.layers:   # non-zero norm weights, so a wrong norm would show
            for k in ("in_norm", "post_norm", "q_norm", "k_norm", "m_in_norm", "m_q_norm", "m_k_norm"):
                if k in L:
                    L[k].copy_(torch.linspace(-0.3, 0.3, L[k].numel()))
        _fill_caches(m, 4)
        models.append(m)
    tokens = torch.tensor([1, 5, 999, 42, 7])
    positions = torch.tensor([20, 63, 64, 100, 5])
    valid = torch.tensor([True, True, True, False, True])
    outs = [m.decode_step(tokens, positions, valid) for m in models]
    err = rel_err(outs[0], outs[1])
    assert err <= 1e-5, err
    for x, y in zip(models[0].cache_tensors(), models[1].cache_tensors()):
        if x.is_floating_point():   # (empty memory slots score -inf in both)
            torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6)
        else:
            assert torch.equal(x, y)


for _name in ("conv_prefill", "swa_prefill", "ring_fill"):
    setattr(TorchGlueOps, _name, staticmethod(getattr(rt.TorchGlue, _name)))


def _small_model(ops=None, seed=3):
    m = rt.Model(_small(), batch=1, device="cpu", seed=seed, ops=ops or HostOps(), dtype=torch.float32)
    for L in m.layers:
        for k in ("in_norm", "post_norm", "q_norm", "k_norm", "m_in_norm", "m_q_norm", "m_k_norm"):
            if k in L:
                L[k].copy_(torch.linspace(-0.3, 0.3, L[k].numel()))
        if "writer_down" in L:   # a live writer, so the memory keys depend on it
            L["writer_down"].normal_(0, 0.02, generator=torch.Generator().manual_seed(7))
    return m


def _prompts(lengths, seed=11):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 1000, (n,), generator=g) for n in lengths]


def _assert_caches_close(a, b, tol=1e-5, live_only=False):
    """Caches in cache_tensors() order equal within ``tol`` (integers
    exactly).  ``live_only``: anchor-memory slots are compared where they hold
    a token (committed slots with a position, pending slots below the count);
    a decode commit leaves stale pending rows that _sequence zeroes, and
    neither is ever read."""
    a, b = list(a), list(b)
    cfg = _small()
    n_gdn = sum(1 for i in range(cfg.layers) if not cfg.is_memory_layer(i))
    mem = []
    k = 2 * n_gdn
    while k < len(a):
        mem.append(k + 3)
        k += 3 + 9
    for j, (x, y) in enumerate(zip(a, b)):
        base = next((m for m in mem if m <= j < m + 9), None)
        if live_only and base is not None:
            field = j - base
            pos, cnt = a[base + 3], a[base + 7]
            if field in (0, 1, 2):      # committed keys / values / scores
                live = pos >= 0
                x, y = x[live], y[live]
            elif field in (4, 5, 6):    # pending keys / values / scores
                slot = torch.arange(x.shape[2])
                live = slot[None, None, :] < cnt[:, None, None]
                live = live.expand(x.shape[:3])
                x, y = x[live], y[live]
        if x.is_floating_point():
            torch.testing.assert_close(x, y, rtol=tol, atol=tol)
        else:
            assert torch.equal(x, y), j


def test_packed_ragged_prefill_equals_per_prompt_prefill():
    """Ragged prompts packed into one pass (cu_seqlens) leave, row by row,
    the logits and caches each prompt leaves alone: lengths around the
    window (64) and the memory chunk (8), one token, and past the window."""
    m = _small_model()
    prompts = _prompts([5, 70, 1, 150, 64, 9])
    logits, caches = m.prefill(prompts)
    for r, p in enumerate(prompts):
        one, alone = m.prefill([p])
        assert rel_err(logits[r], one[0]) <= 1e-5, r
        _assert_caches_close([c[r: r + 1] for c in caches], alone)


def test_pieced_prefill_equals_whole_prefill():
    """A prompt taken in pieces (each continuing the GDN state, the conv
    window, the ring as left context and the memory through _sequence with a
    state) equals the whole prompt at once; pieces of 7, 32 and 64 tokens,
    rows of different lengths finishing in different pieces."""
    m = _small_model()
    prompts = _prompts([150, 37, 100], seed=12)
    logits, caches = m.prefill(prompts)
    for piece in (7, 32, 64):
        lp, cp = m.prefill(prompts, token_chunk=piece)
        assert rel_err(lp, logits) <= 1e-5, piece
        _assert_caches_close(cp, caches)


def test_prefill_then_decode_equals_longer_prefill():
    """Prefill of T tokens then one decode step equals the prefill of T + 1
    tokens (logits and every cache), T past the window and the memory's
    chunks, and T + 1 a memory commit: the prefill leaves the ring and the
    anchor memory as the decode path reads them."""
    m = _small_model()
    for t in (70, 79, 130):
        p = _prompts([t + 1], seed=t)[0]
        ref_logits, ref_caches = m.prefill([p])
        _, caches = m.prefill([p[:t]])
        m.B = 1
        m._alloc_caches()
        for dst, src in zip(m.cache_tensors(), caches):
            dst.copy_(src)
        out = m.decode_step(p[t:t + 1], torch.tensor([t]), torch.tensor([True]))
        assert rel_err(out, ref_logits) <= 1e-5, t
        _assert_caches_close(m.cache_tensors(), ref_caches, live_only=True)


def test_prefill_host_ops_match_the_runtime_torch_glue():
    """The prefill through HostOps equals the prefill through the runtime's
    torch forms of the prefill glue (conv continuation, window attention
    with the ring as context, ring fill) on ragged, pieced prompts."""
    prompts = _prompts([90, 3, 41], seed=13)
    outs = []
    for ops in (HostOps(), TorchGlueOps()):
        m = _small_model(ops)
        outs.append(m.prefill(prompts, token_chunk=32))
    assert rel_err(outs[0][0], outs[1][0]) <= 1e-5
    _assert_caches_close(outs[0][1], outs[1][1])
