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
