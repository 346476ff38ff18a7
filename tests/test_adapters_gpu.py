"""The vLLM / SGLang anchor-memory layer on ROCm (yanchor_amd/adapters.py)
against the oracle (GPU).

A vLLM batch mixes decode rows (one token each, one of them a padding row
with state index -1) and prefill spans (one starting at position 0, which
resets its slot, one continuing a slot's memory).  The projections the layer
computes are handed to the oracle's restatement of the reference's memory
operations (committed read + push / commit for decode tokens, ``_sequence``
with a state for prefill spans): every slot page is bit-exact after the
call, untouched slots unchanged, and the gated reads are within 1e-2 of the
float64 oracle.  SGLang's ``MemorySlots`` lifecycle (reset, copy, CPU
offload and load) and its decode / extend forward are checked the same way.

Both layers are called as the reference's are: ``forward(hidden, positions)``
with the metadata in the forward context (vllm_yanchor.py:66-97) and
``forward(hidden, positions, forward_batch)`` with the request-to-token pool
(sglang_models/yanchor.py:53-83); the framework objects are stand-ins holding
exactly the fields the reference layers read.
"""
from dataclasses import fields
from types import SimpleNamespace

import pytest
import torch

from oracle import anchor as ref
from yanchor_amd import adapters, slot_pages, workloads
from yanchor_amd import runtime as rt
from yanchor_amd.independent_memory import IndependentMemoryState

from conftest import rel_err

pytestmark = pytest.mark.gpu

LAYER = 3


def small_cfg():
    return rt.ModelConfig(layers=4, hidden=256, intermediate=512, vocab=1000, gdn_heads_k=2, gdn_heads_v=4,
                          attn_heads=8, kv_heads=2, head_dim=128, rotary_dim=32, swa_window=128,
                          memory_capacity=64, memory_chunk=8, writer_intermediate=256, admission_rank=16,
                          init_std=0.05)


def _row(st, i):
    """One row of a memory state as an oracle state on the host."""
    return ref.MemoryState(*(getattr(st, f.name)[i:i + 1].cpu().clone() for f in fields(st)))


def _assert_row_equal(got, i, want, what):
    for f in fields(want):
        a, b = getattr(got, f.name)[i:i + 1].cpu(), getattr(want, f.name)
        assert torch.equal(a, b), f"{what}: slot field {f.name} differs"


def _oracle_decode(layer, proj, r, state_row):
    q, gate, key, value, scores = (x[r:r + 1].cpu() for x in proj)
    read = ref.committed_read(q[:, None], state_row)[:, 0]
    ref.commit_decode(key[:, None], value[:, None], scores[:, None], torch.tensor([True]), layer.chunk, state_row)
    return read * gate[..., None].double()


def _oracle_sequence(layer, proj, state_row):
    q, gate, key, value, scores = (x.cpu() for x in proj)
    read = ref.sequence(q, key, value, scores, None, layer.chunk, state_row)
    return (read * gate[..., None].double())[0]


def test_vllm_mixed_batch_matches_oracle(gpu):
    cfg = small_cfg()
    m = rt.Model(cfg, batch=1, device=gpu, seed=9)
    context = SimpleNamespace(attn_metadata=None)
    layer = adapters.VllmMemory(m, LAYER, prefix="model.layers.3.memory", forward_context=lambda: context)
    g, cap, c, d = cfg.kv_heads, cfg.memory_capacity, layer.chunk, cfg.head_dim
    slots = 8
    pages = slot_pages.empty_pages(slots, g, cap, c, d, gpu, torch.bfloat16)
    init = workloads.anchor_state(slots, g, cap, c, d, seed=11, fill_pending=5)
    view = layer.state(pages)
    for f in fields(init):
        getattr(view, f.name).copy_(getattr(init, f.name))
    before = IndependentMemoryState(*(getattr(view, f.name).clone() for f in fields(view)))
    # decode rows: slots 5, padding, 2; prefill: slot 7 from position 0 (70
    # tokens), slot 0 continuing its memory (21 tokens)
    idx = torch.tensor([5, -1, 2, 7, 0], dtype=torch.int32)
    lens = [1, 1, 1, 70, 21]
    starts = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    total0 = int(init.total[0])
    positions = torch.cat([torch.tensor([300, 0, 77]), torch.arange(70), total0 + torch.arange(21)]).to(gpu)
    hidden = (torch.randn(sum(lens), cfg.hidden, generator=torch.Generator().manual_seed(12)) * 0.5).to(
        torch.bfloat16).to(gpu)
    meta = adapters.VllmMetadata(num_decodes=3, num_prefills=2, non_spec_state_indices_tensor=idx.to(gpu),
                                 non_spec_query_start_loc=starts.to(gpu))
    context.attn_metadata = {layer.prefix: meta}
    layer.kv_cache = pages
    # the reference's call (three equal M-RoPE rows, as vLLM may pass them)
    out = layer.forward(hidden, positions[None].expand(3, -1))
    torch.cuda.synchronize()
    # the same batch through run() on a copy of the starting pages gives the reads
    pages2 = slot_pages.empty_pages(slots, g, cap, c, d, gpu, torch.bfloat16)
    view2 = layer.state(pages2)
    for f in fields(before):
        getattr(view2, f.name).copy_(getattr(before, f.name))
    out2, reads = layer.run(hidden, positions, meta, pages2, return_reads=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    for f in fields(before):
        assert torch.equal(getattr(view, f.name), getattr(view2, f.name)), f.name
    assert out.shape == hidden.shape and torch.isfinite(out.float()).all()
    # the oracle on the layer's own projections
    dec = layer.project_decode(hidden[:3], positions[:3])
    for r, slot in ((0, 5), (2, 2)):
        st = _row(before, slot)
        want = _oracle_decode(layer, dec, r, st)
        assert rel_err(reads[r:r + 1], want) <= 1e-2, (slot, rel_err(reads[r:r + 1], want))
        _assert_row_equal(view, slot, st, f"decode slot {slot}")
    assert not reads[1].any()                                      # the padding row reads nothing
    spans = ((3, 73, 7, True), (73, 94, 0, False))
    for lo, hi, slot, fresh in spans:
        st = ref.MemoryState.empty(1, g, cap, c, d) if fresh else _row(before, slot)
        want = _oracle_sequence(layer, layer.project_sequence(hidden[lo:hi], positions[lo:hi]), st)
        err = rel_err(reads[lo:hi], want)
        print(f"prefill slot {slot} ({hi - lo} tokens, fresh={fresh}): read rel err {err:.2e}", flush=True)
        assert err <= 1e-2
        _assert_row_equal(view, slot, st, f"prefill slot {slot}")
    for slot in (1, 3, 4, 6):
        _assert_row_equal(view, slot, _row(before, slot), f"untouched slot {slot}")
    # the layer's output is the memory output projection of the gated reads
    assert rel_err(out, torch.nn.functional.linear(reads.flatten(-2), m.layers[LAYER]["m_o"])) <= 1e-2
    # no metadata (vLLM's profiling run): one sequence over a fresh memory, pages untouched
    context.attn_metadata = None
    snapshot = [getattr(view, f.name).clone() for f in fields(view)]
    fresh = layer.forward(hidden[3:73], positions[3:73])
    torch.cuda.synchronize()
    assert torch.equal(fresh, out[3:73])
    for f, t in zip(fields(view), snapshot):
        assert torch.equal(getattr(view, f.name), t), f.name


class _ReqToTokenPool:
    """The part of SGLang's request-to-token pool the memory layer reads:
    ``mamba_pool`` (size, slot-state registration) and the request-to-row
    index maps."""

    def __init__(self, size, rows):
        self.registered = []
        self.mamba_pool = SimpleNamespace(size=size, register_slot_state=self.registered.append)
        self.rows = rows

    def get_mamba_indices(self, req_pool_indices):
        return self.rows[req_pool_indices.long()]

    def translate_mamba_indices(self, indices):
        return indices


def _forward_batch(decode, req_pool_indices, seq_lens=None, prefix_lens=None):
    return SimpleNamespace(forward_mode=SimpleNamespace(is_decode=lambda: decode), req_pool_indices=req_pool_indices,
                           extend_seq_lens_cpu=seq_lens, extend_prefix_lens_cpu=prefix_lens)


def test_sglang_slots_lifecycle_and_forward(gpu):
    cfg = small_cfg()
    m = rt.Model(cfg, batch=1, device=gpu, seed=13)
    # request pool index r lives on memory row rows[r]
    pool = _ReqToTokenPool(6, torch.tensor([2, 4, 0, 5, 3, 1], device=gpu))
    layer = adapters.SglangMemory(m, LAYER, req_to_token_pool=lambda: pool)
    g, cap, c, d = cfg.kv_heads, cfg.memory_capacity, layer.chunk, cfg.head_dim
    # the first call creates and registers the slots: an extend of one new request on row 3
    pos = torch.arange(25, device=gpu)
    hidden = (torch.randn(25, cfg.hidden, generator=torch.Generator().manual_seed(17)) * 0.5).to(
        torch.bfloat16).to(gpu)
    layer.forward(hidden, pos, _forward_batch(False, torch.tensor([4], device=gpu), [25], [0]))
    torch.cuda.synchronize()
    slots = layer.slots
    assert pool.registered == [slots] and slots.layer_id == LAYER
    assert slots.state.keys.shape[0] == 7                          # size + 1 rows
    st = ref.MemoryState.empty(1, g, cap, c, d)
    _oracle_sequence(layer, layer.project_sequence(hidden, pos), st)
    _assert_row_equal(slots.state, 3, st, "first extend row 3")
    init = workloads.anchor_state(7, g, cap, c, d, seed=14, fill_pending=3)
    for f in fields(init):
        getattr(slots.state, f.name).copy_(getattr(init, f.name))
    # lifecycle: copy 1 -> 4, offload 2 and load it into 5, reset 3
    slots.copy_slots(torch.tensor([1]), torch.tensor([4]))
    data = slots.get_cpu_slots(torch.tensor([2]))
    slots.load_cpu_slots(data, torch.tensor([5]))
    slots.reset_slots(torch.tensor([3]))
    for f in fields(init):
        t = getattr(slots.state, f.name).cpu()
        src = getattr(init, f.name)
        assert torch.equal(t[4], src[1]) and torch.equal(t[5], src[2]), f.name
        assert torch.equal(t[0], src[0]) and torch.equal(t[6], src[6]), f.name
    assert bool((slots.state.positions[3] == -1).all()) and int(slots.state.count[3]) == 0
    names = [n for n, *_ in slots.iter_transfer_state_entries()]
    assert names == [f"yanchor_{f.name}" for f in fields(init)]
    before = IndependentMemoryState(*(getattr(slots.state, f.name).clone() for f in fields(slots.state)))
    # decode: requests 1, 2, 3 on rows 4, 0, 5
    rows = [4, 0, 5]
    pos = torch.tensor([40, 41, 42], device=gpu)
    hidden = (torch.randn(3, cfg.hidden, generator=torch.Generator().manual_seed(15)) * 0.5).to(
        torch.bfloat16).to(gpu)
    dec = layer.project_decode(hidden, pos)
    out = layer.forward(hidden, pos, _forward_batch(True, torch.tensor([1, 2, 3], device=gpu)))
    torch.cuda.synchronize()
    assert out.shape == hidden.shape
    for r, row in enumerate(rows):
        st = _row(before, row)
        _oracle_decode(layer, dec, r, st)
        _assert_row_equal(slots.state, row, st, f"decode row {row}")
    # extend: request 4 on row 3 (reset, prefix 0) 30 tokens, request 5 on row 1 (continuing) 12 tokens
    before = IndependentMemoryState(*(getattr(slots.state, f.name).clone() for f in fields(slots.state)))
    lens, prefix = [30, 12], [0, int(before.total[1])]
    pos = torch.cat([torch.arange(30), prefix[1] + torch.arange(12)]).to(gpu)
    hidden = (torch.randn(42, cfg.hidden, generator=torch.Generator().manual_seed(16)) * 0.5).to(
        torch.bfloat16).to(gpu)
    out = layer.forward(hidden, pos, _forward_batch(False, torch.tensor([4, 5], device=gpu), lens, prefix))
    torch.cuda.synchronize()
    for (lo, hi), row, fresh in (((0, 30), 3, True), ((30, 42), 1, False)):
        st = ref.MemoryState.empty(1, g, cap, c, d) if fresh else _row(before, row)
        _oracle_sequence(layer, layer.project_sequence(hidden[lo:hi], pos[lo:hi]), st)
        _assert_row_equal(slots.state, row, st, f"extend row {row}")


def test_adapter_getters_fail_loudly_without_framework(gpu):
    m = rt.Model(small_cfg(), batch=1, device=gpu, seed=3)
    hidden = torch.zeros(2, m.cfg.hidden, device=gpu, dtype=torch.bfloat16)
    pos = torch.arange(2, device=gpu)
    with pytest.raises(RuntimeError, match="forward context"):
        adapters.VllmMemory(m, LAYER).forward(hidden, pos)
    with pytest.raises(RuntimeError, match="request-to-token pool"):
        adapters.SglangMemory(m, LAYER).forward(hidden, pos, _forward_batch(True, torch.tensor([0, 1], device=gpu)))
