"""The reference's generation API (runtime/inference.py:23-125) on the HIP
decode path, small random model (GPU).

* ``Engine.generate`` returns every row, sorted by attempt id, with the
  reference's output keys, and metrics with the reference's keys;
* with ``fixed`` (no EOS) every row generates exactly its cap (the global
  ``cap`` or a smaller per-row ``max_tokens``: finish reason
  "prompt_length_cap");
* more prompts than slots: finished slots are refilled from the stream, and
  each row's tokens equal those of a run with a different slot count
  (float32 model, argmax: rows do not interact);
* ``on_tokens`` sees exactly each row's response ids;
* a row whose first token is an EOS id finishes with reason "eos" after one
  token; temperature 0 is the argmax;
* the eager backend ("torch") gives the graph backend's tokens.
"""
import pytest
import torch

from yanchor_amd import inference
from yanchor_amd import runtime as rt

pytestmark = pytest.mark.gpu

ROW_KEYS = {"attempt_id", "sample_index", "max_tokens", "checkpoint_id", "protocol_key", "response", "response_ids",
            "generated_tokens", "prompt_tokens", "finish_reason", "finished_by_eos", "cap_hit"}
METRIC_KEYS = {"decode_useful_token_events", "generation_wall_seconds", "initial_prefill_seconds",
               "refill_prefill_seconds", "decode_seconds", "decode_tokens_per_second", "peak_allocated_gib",
               "model_load_seconds", "operators", "physical_slots", "refilled_attempts", "tail_compaction_shapes",
               "stream_committed_groups"}


def small_cfg(**kw):
    base = dict(layers=8, hidden=256, intermediate=512, vocab=1000, gdn_heads_k=2, gdn_heads_v=4,
                attn_heads=8, kv_heads=2, head_dim=128, rotary_dim=32, swa_window=128, memory_capacity=64,
                memory_chunk=8, writer_intermediate=256, admission_rank=16, init_std=0.05)
    base.update(kw)
    return rt.ModelConfig(**base)


def test_profiles_pick_the_state_storage(gpu):
    """As the reference's engine (runtime/inference.py:53-56): profile "fast"
    keeps the GDN state in float16 for batches above one, "reference", one
    row or the eager torch backend in float32; the fast engine generates."""
    cfg = small_cfg(gdn_heads_k=4, gdn_heads_v=4)
    for kw, want in ((dict(batch=4), torch.float16), (dict(batch=4, profile="reference"), torch.float32),
                     (dict(batch=1), torch.float32), (dict(batch=4, backend="torch"), torch.float32)):
        eng = inference.Engine(cfg, device=gpu, **kw)
        assert eng.model.state_dtype == want, kw
        assert eng.operators["recurrent_state"] == str(want).removeprefix("torch."), kw
        assert all(x.dtype == want for x in eng.model.gdn_state.values())
    eng = inference.Engine(cfg, device=gpu, batch=4)
    rows = [dict(input_ids=p, max_tokens=12) for p in _prompts(6, seed=3)]
    out, met = eng.generate(rows, cap=12, fixed=True, stop_interval=4)
    assert [r["attempt_id"] for r in out] == list(range(6))
    assert all(1 <= len(r["response_ids"]) <= 12 for r in out)


def _prompts(n, seed=1, lo=5, hi=40):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi, (n,), generator=g).tolist()
    return [torch.randint(0, 1000, (L,), generator=g).tolist() for L in lens]


def test_generate_rows_metrics_and_caps(gpu):
    m = rt.Model(small_cfg(), batch=4, device=gpu, seed=2)
    eng = inference.Engine(m, batch=4)
    prompts = _prompts(9)
    rows = [dict(input_ids=p, max_tokens=(7 if i % 3 == 0 else 50)) for i, p in enumerate(prompts)]
    seen = {}

    def on_tokens(aid, toks):
        seen.setdefault(aid, []).extend(toks)

    out, met = eng.generate(rows, on_tokens=on_tokens, cap=24, fixed=True, stop_interval=8)
    assert [r["attempt_id"] for r in out] == list(range(9))
    for i, r in enumerate(out):
        assert ROW_KEYS <= set(r), ROW_KEYS - set(r)
        want = 7 if i % 3 == 0 else 24
        assert r["generated_tokens"] == len(r["response_ids"]) == want, (i, r["generated_tokens"])
        assert r["finish_reason"] == ("prompt_length_cap" if i % 3 == 0 else "length")
        assert r["prompt_tokens"] == len(prompts[i]) and r["cap_hit"] and not r["finished_by_eos"]
        assert all(0 <= t < 1000 for t in r["response_ids"])
        assert seen[i] == r["response_ids"]
    assert METRIC_KEYS <= set(met), METRIC_KEYS - set(met)
    assert met["physical_slots"] == 4 and met["refilled_attempts"] == 5
    assert met["stream_committed_groups"] == 9
    # useful events: every token after each row's first (reference inference.py:105-106)
    assert met["decode_useful_token_events"] == sum(r["generated_tokens"] - 1 for r in out)
    assert met["decode_tokens_per_second"] > 0


def test_rows_do_not_depend_on_slot_count(gpu):
    """float32 activations and argmax sampling: a row's tokens are the same
    whether 2 or 5 slots run, refills and compactions included."""
    prompts = _prompts(6, seed=3)
    outs = []
    for batch in (2, 5):
        m = rt.Model(small_cfg(), batch=batch, device=gpu, seed=4, dtype=torch.float32)
        eng = inference.Engine(m, batch=batch)
        out, met = eng.generate(prompts, cap=20, temperature=0.0, stop_interval=4)
        outs.append([r["response_ids"] for r in out])
    assert outs[0] == outs[1]


def test_eos_first_token_and_argmax(gpu):
    """temperature 0 is the argmax (inference.py:82-83); a row whose first
    token is an EOS id finishes at once with reason "eos"."""
    m = rt.Model(small_cfg(), batch=3, device=gpu, seed=5)
    prompts = _prompts(3, seed=6, lo=10, hi=11)            # one length: one prefill
    logits, _ = m.prefill(torch.tensor(prompts, device=gpu))
    first = logits.argmax(-1).tolist()
    eng = inference.Engine(m, batch=3)
    out, _ = eng.generate(prompts, cap=16, temperature=0.0, eos_ids=(first[1], 999999), stop_interval=4)
    assert out[1]["finish_reason"] == "eos" and out[1]["generated_tokens"] == 1 and out[1]["finished_by_eos"]
    for i in (0, 2):
        assert out[i]["response_ids"][0] == first[i]
        assert out[i]["finish_reason"] in ("eos", "length", "mechanical_repetition")


@pytest.mark.parametrize("top_k,top_p", [(20, 0.95), (0, 1.0), (100, 0.9)])
def test_eager_backend_matches_graph(gpu, top_k, top_p):
    """The eager loop ("torch" backend) replays what the captured graph
    does; top_k != 20 switches to the torch sampler, top_k <= 0 / > 64 to its
    full-vocabulary branches."""
    prompts = _prompts(5, seed=7)
    outs = []
    for backend in ("hip", "torch"):
        m = rt.Model(small_cfg(), batch=3, device=gpu, seed=8)
        eng = inference.Engine(m, batch=3, backend=backend)
        out, met = eng.generate(prompts, cap=12, top_k=top_k, top_p=top_p, presence_penalty=1.5, fixed=True,
                                stop_interval=4)
        outs.append([r["response_ids"] for r in out])
        assert met["backend"] == backend
    assert outs[0] == outs[1]
