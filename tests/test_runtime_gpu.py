"""End-to-end checks of the decode runtime on a small random model (GPU).

* decode after prefill reproduces prefill of one more token (every cache --
  GDN state, conv window, SWA ring, anchor memory -- is consistent between the
  two paths): last-token logits within 1e-4 relative error in float32, 5e-2
  with bf16 activations (different GEMM shapes round differently);
* the captured HIP graph of the decode step reproduces eager steps exactly,
  over several replays with eager work and synchronisations in between;
* a short continuous-batching run keeps its accounting consistent.
"""
import copy

import pytest
import torch

from yanchor_amd import runtime as rt

from conftest import rel_err

pytestmark = pytest.mark.gpu


def small_cfg(**kw):
    base = dict(layers=8, hidden=256, intermediate=512, vocab=1000, gdn_heads_k=2, gdn_heads_v=4,
                attn_heads=8, kv_heads=2, head_dim=128, rotary_dim=32, swa_window=128, memory_capacity=64,
                memory_chunk=8, writer_intermediate=256, admission_rank=16, init_std=0.05)
    base.update(kw)
    return rt.ModelConfig(**base)


@pytest.mark.parametrize("dtype,tol,b,over", [
    (torch.float32, 1e-4, 3, {}), (torch.bfloat16, 5e-2, 3, {}),
    # as many key heads as value heads (the fused GDN decode core), more than
    # 128 slots (projections past the packed kernel's rows), a 16-slot memory
    (torch.bfloat16, 5e-2, 130, {"gdn_heads_k": 4, "memory_capacity": 16})])
def test_decode_after_prefill_matches_longer_prefill(gpu, dtype, tol, b, over):
    """fp32 pins the cache logic tightly; bf16 bounds the rounding drift."""
    cfg = small_cfg(**over)
    m = rt.Model(cfg, batch=b, device=gpu, seed=1, dtype=dtype)
    g = torch.Generator().manual_seed(2)
    prompts = torch.randint(0, cfg.vocab, (b, 21), generator=g).to(gpu)
    ref_logits, _ = m.prefill(prompts)                      # 21 tokens
    logits, caches = m.prefill(prompts[:, :20])              # 20 tokens ...
    for dst, src in zip(m.cache_tensors(), caches):
        dst.copy_(src)
    pos = torch.full((b,), 20, dtype=torch.long, device=gpu)
    valid = torch.ones(b, dtype=torch.bool, device=gpu)
    out = m.decode_step(prompts[:, 20], pos, valid)          # ... plus one decode step
    torch.cuda.synchronize()
    assert rel_err(out, ref_logits) <= tol, rel_err(out, ref_logits)


def test_graph_replay_matches_eager(gpu):
    cfg = small_cfg()
    m = rt.Model(cfg, batch=4, device=gpu, seed=3)
    eng = rt.Engine(m, poll_interval=4, max_rows=64, max_new_tokens=64)
    eng.capture()
    reqs = rt.synthetic_requests(1, rate=4, prompt_len=16, mean_len=20, max_len=64, vocab=cfg.vocab, seed=4)
    reqs = (reqs * 4)[:4]
    for i, r in enumerate(reqs):
        r.attempt_id = i
    eng.admit(reqs, [0, 1, 2, 3])
    # eager twin of the whole engine state
    twin = rt.Engine.__new__(rt.Engine)
    twin.__dict__.update({k: (v.clone() if torch.is_tensor(v) else v) for k, v in eng.__dict__.items()})
    twin.m = copy.copy(m)
    twin.m._alloc_caches()
    for dst, src in zip(twin.m.cache_tensors(), m.cache_tensors()):
        dst.copy_(src)
    twin.use_graph, twin.graph = False, None
    for step in range(6):
        eng.step()
        twin.step()
        torch.cuda.synchronize()
        assert torch.equal(eng.decode_ids, twin.decode_ids), step
        assert torch.equal(eng.finished, twin.finished) and torch.equal(eng.useful, twin.useful)
        for a, b in zip(eng.m.cache_tensors(), twin.m.cache_tensors()):
            assert torch.equal(a, b)
        _ = torch.randn(1000, device=gpu).sum().item()  # unrelated eager work between replays


def test_short_engine_run(gpu):
    cfg = small_cfg()
    m = rt.Model(cfg, batch=8, device=gpu, seed=5)
    met = rt.run_decode_benchmark(m, steps=40, warmup=8, rate=2.0, prompt_len=16, mean_len=12, poll_interval=4,
                                  max_new_tokens=64)
    assert met.decode_steps == 40
    assert 0 < met.decode_useful_token_events <= met.decode_scheduled_token_events
    assert met.decode_seconds > 0 and met.decode_tokens_per_second > 0


def test_tail_compaction_keeps_every_sequence(gpu):
    """Shrinking the physical batch mid-generation (live slots gathered in
    ascending order, graph captured again) leaves every sequence's tokens and
    length as in a run without compaction (float32, so the smaller GEMMs do
    not change the sampled tokens)."""
    cfg = small_cfg()
    g = torch.Generator().manual_seed(9)
    caps = [3, 5, 9, 20, 31, 40]
    reqs = [rt.Request(i, torch.randint(0, cfg.vocab, (16,), generator=g), c, 0) for i, c in enumerate(caps)]
    out = []
    for compact in (False, True):
        m = rt.Model(cfg, batch=8, device=gpu, seed=3, dtype=torch.float32)
        eng = rt.Engine(m, poll_interval=4, max_rows=16, max_new_tokens=64, tail_compaction=compact)
        met = rt.run_decode_benchmark(m, steps=56, warmup=0, poll_interval=4, requests=copy.deepcopy(reqs),
                                      engine=eng)
        assert met.extra["live_slots_end"] == 0
        out.append((eng.outputs(), met.extra["tail_compactions"]))
    (o0, c0), (o1, c1) = out
    assert c0 == [] and len(c1) >= 1 and all(0 < x < 8 for x in c1), c1
    assert sorted(o0) == sorted(o1) == list(range(len(caps)))
    for i, c in enumerate(caps):
        assert len(o0[i]) == len(o1[i]) == c, i
        assert o0[i] == o1[i], i
