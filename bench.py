"""Benchmark of the YANchor recurrent decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Prints one JSON line.  Workloads:

* ``model_decode`` (default): continuous-batching decode of the random-init
  4B-shaped hybrid model (36 layers: 27 Gated DeltaNet + 9 sliding-window /
  anchor-memory layers, hidden 2560, 32 heads, dk = dv = 128, 256 anchor slots,
  vocab 151936, bf16 weights ~ N(0, 0.02)) over a physical batch of 128 slots.
  One request per slot is queued before the first step and prefilled into the
  batch (the reference's initial fill); then requests arrive as a Poisson
  process (mean 4 per step) with random 128-token prompts and geometric
  generation lengths (mean 1024); finished slots are refilled at poll points
  every 32 steps and once more before the timed window, so it starts with
  every slot live; sampling is top-k 20 / top-p 0.95 /
  T = 0.6 with presence penalty 1.5.  One step = one captured HIP graph of the
  whole model forward + sampling + slot bookkeeping for all 128 slots.
  value = useful decode tokens / (timed wall - refill prefill time), the
  reference's decode tokens/s definition; ``decode.live_slots`` gives the
  live slots per timed step (min / mean / first / last), ``decode.ring_fill``
  the mean live fraction of the SWA rings those steps read (a young ring is
  cheaper: the window read skips blocks without a live slot).  Beside the
  decode line the same run reports ``fp16_state`` (the same workload with the
  GDN state stored in float16, the reference's "fast" profile; not the line's
  value, whose state is float32), ``prefill`` (the ``gdn_prefill`` workload:
  20 timed calls after 20 warm-up calls, with its HBM and MFMA roofline) and
  ``sampling`` (the ``sampling`` workload at the decode batch).
* ``long_horizon``: B=256 fixed sequences generating 32768 tokens from
  256-token prompts, 16-slot anchor memory committed every 64 tokens;
  sustained tokens/s over a bounded window of steps and peak HBM use.
* ``gdn_decode``: the state-update kernel alone on a [B, 32, 128, 128] fp32
  state (``--batch``, default 64) with bf16 q/k/v, cycling over 4 layer states.
* ``gdn_decode_fused``: the model's per-layer GDN decode core (conv window
  update, state update, gated norm; ``--batch``, default 128), 4 rotating
  layers.
* ``gdn_prefill``: varlen chunked prefill of one GDN layer on the MFMA chunk
  kernel (32 packed sequences, lengths U[512, 8192]); reports MFMA utilisation
  beside the HBM fraction.
* ``anchor_prefill``: the anchor-memory half of a prefill that continues a
  state (32 rows x 2048 tokens, 8 memories of 256 slots, C = 64), and its
  MFMA block read alone.
* ``sampling``: the decode step's sampler (fused top-20 semantics, top-p 0.95,
  presence penalty) on 128 rows of bf16 logits over the full vocabulary.
* ``projections``: every decode projection of the model at M = 128 on the
  packed-weight kernels, as the step calls them, beside hipBLASLt.
* ``hbm_copy``: a 128 MiB device copy, the calibration kernel for the HBM byte
  counters behind ``roofline.traffic``; ``hbm_streams_gbs`` adds the rates of
  the library's calibration streams (copy, in-place read-modify-write, read,
  write; plain and nontemporal) over 1 GiB buffers, ``gemm_bf16`` the rate of
  an 8192^3 bf16 library GEMM beside the 2.5 PFLOP/s MFMA spec.

Timing: W untimed steps, then K steps between two device synchronisations.
``roofline`` prices the fused GDN decode core (the dominant hot-path kernel:
conv window update, state update and gated norm of one GDN layer): its
algorithmic bytes per launch at the model's decode shape over its average
launch time, measured here with HIP events on the stream the kernel runs on,
cycling over the model's 27 GDN layers.  ``cpu_baseline`` runs the same
model's decode step on the host cores with every op from the oracle
(oracle/model_ops.py: recurrence, anchor memory, ring attention, layer glue,
sampler), on a bounded number of steps.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "decode tokens/s at B=128 on 1 GPU; state-update HBM GB/s as % of peak"
# HBM bytes per launch of gdn_recurrent_kernel, by batch rows, from rocprofv3
# --pmc FETCH_SIZE and WRITE_SIZE (KiB per dispatch) on
# ``bench.py --workload gdn_decode --batch B``, scaled by what the same counters
# read for a 128 MiB float4 copy kernel (FETCH x 2.0, WRITE x 1.0).
TRAFFIC_GDN_DECODE = {128: (133803.7 * 2.0 + 263283.8) * 1024}
# The same for gdn_decode_fused_kernel (``--workload gdn_decode_fused``), by batch rows.
TRAFFIC_GDN_FUSED = {128: (137924.0 * 2.0 + 272580.8) * 1024}
TRAFFIC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this kernel at this shape, scaled by the "
                  "copy-kernel factors (FETCH x 2.0, WRITE x 1.0); a constant, not measured in this run")
# The same for one call of the chunked prefill (``--workload gdn_prefill``,
# chunk_fused_kernel).
TRAFFIC_PREFILL = (2074512.6 * 2.0 + 1341736.0) * 1024
# The same for one anchor read (``--workload anchor_read``, 64 x 32 x 256 x 128).
TRAFFIC_ANCHOR_READ = (97995.3 * 2.0 + 512.0) * 1024


def gdn_state_bytes(b, h, hv, kd, vd, qkv_size, gate_size, with_indices):
    """Algorithmic HBM bytes of one decode step of the state update."""
    state = 2 * b * hv * kd * vd * 4                 # fp32 state read + write
    inputs = b * (2 * h * kd + hv * vd) * qkv_size   # q, k, v
    gates = 2 * b * hv * gate_size                   # g, beta
    out = b * hv * vd * qkv_size                     # o
    idx = 4 * b if with_indices else 0
    return state + inputs + gates + out + idx


def gdn_fused_bytes(b, hv, d, conv_dim):
    """Algorithmic HBM bytes of one decode step of the fused GDN layer core:
    the fp32 state read + write, the projection row read (conv channels, z,
    b, a), the conv window read + write, the conv weights, the output row."""
    state = 2 * b * hv * d * d * 4
    proj = b * (conv_dim + hv * d + 2 * hv) * 2
    window = 2 * b * 3 * conv_dim * 2
    return state + proj + window + conv_dim * 4 * 2 + b * hv * d * 2


def _fused_step(dev, b, hv, d, conv_dim, layers_in, seed):
    """Launch closure of the fused GDN decode core over rotating layers;
    ``layers_in`` = [(conv_state, conv_w, a_log, dt_bias, state, norm_w)]."""
    from yanchor_amd import layers

    vd = hv * d
    g = torch.Generator(device=dev).manual_seed(seed)
    proj = torch.randn(b, conv_dim + vd + 2 * hv, device=dev, generator=g).to(torch.bfloat16)

    def step(i):
        conv, conv_w, a_log, dt_bias, state, norm_w = layers_in[i % len(layers_in)]
        layers.gdn_decode_fused(proj, conv, conv_w, a_log, dt_bias, state, norm_w, 1e-6, heads=hv, head_dim=d,
                                z_offset=conv_dim, b_offset=conv_dim + vd, a_offset=conv_dim + vd + hv)
    return step


def _log(msg):
    """Progress line on stderr (stdout carries only the JSON result)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _affinity() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_threads() -> int:
    """Host threads for the CPU legs: the CPUs this process may run on,
    limited by ``OMP_NUM_THREADS`` when the environment declares the job's CPU
    share that way (a one-GPU job's share of a shared host)."""
    n = _affinity()
    declared = os.environ.get("OMP_NUM_THREADS", "")
    if declared.isdigit() and int(declared) > 0:
        n = min(n, int(declared))
    return max(1, n)


def cpu_host_info() -> dict:
    """What the CPU legs ran on: logical CPUs, the affinity set, the declared
    thread share, torch's thread count and the CPU model name."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "affinity_cpus": _affinity(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "torch_threads": torch.get_num_threads(),
            "cpu_model": model}


def _time_launches(step, steps, warmup):
    """W untimed calls, then K calls between stream synchronisations, with HIP
    events on the current stream (the one the kernels are launched on).
    Returns (wall ms per call, event ms per call)."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        step(warmup + i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall * 1e3 / steps, ev0.elapsed_time(ev1) / steps


def gdn_fused_roofline(model, launches=216, warmup=27):
    """Average launch time of the model's fused GDN decode core (the kernel
    the decode step runs per GDN layer) cycling over the model's GDN layers
    with a fresh bf16 projection row; returns the roofline object."""
    c, b = model.cfg, model.B
    hv, d = c.gdn_heads_v, c.gdn_dv
    ids = sorted(model.gdn_state)
    layers_in = [(model.conv_state[i], model.layers[i]["conv_w"], model.layers[i]["a_log"], model.layers[i]["dt_bias"],
                  model.gdn_state[i], model.layers[i]["gnorm"]) for i in ids]
    step = _fused_step(model.device, b, hv, d, c.conv_dim, layers_in, seed=7)
    _, ms = _time_launches(step, launches, warmup)
    nbytes = gdn_fused_bytes(b, hv, d, c.conv_dim)
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": TRAFFIC_GDN_FUSED.get(b),
            "traffic_source": TRAFFIC_SOURCE if b in TRAFFIC_GDN_FUSED else None,
            "kernel": "gdn_decode_fused_kernel", "bytes_per_launch": nbytes, "avg_launch_us": ms * 1e3,
            "launches": launches,
            "shape": f"state fp32 [{b}, {hv}, {d}, {d}] + conv window bf16 [{b}, 3, {c.conv_dim}], "
                     f"{len(layers_in)} rotating layers"}


def gdn_roofline(states, b, h, kd, vd, launches=216, warmup=27):
    """Average launch time of the GDN decode state update cycling over
    ``states`` (each [b, HV, kd, vd] fp32, updated in place) with fresh bf16
    q/k/v and fp32 gates; returns the roofline object."""
    from yanchor_amd import gdn, workloads

    hv = states[0].shape[1]
    x = workloads.gdn_inputs(b, 1, h, hv, kd, vd, dtype=torch.bfloat16, seed=workloads.SEED0 + 7)
    q, k, v, g, beta = (t.to(states[0].device) for t in (x.q, x.k, x.v, x.g, x.beta))

    def step(i):
        gdn.recurrent_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state=states[i % len(states)])

    _, ms = _time_launches(step, launches, warmup)
    nbytes = gdn_state_bytes(b, h, hv, kd, vd, 2, 4, False)
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": TRAFFIC_GDN_DECODE.get(b),
            "kernel": "gdn_recurrent_kernel", "bytes_per_launch": nbytes, "avg_launch_us": ms * 1e3,
            "launches": launches, "shape": f"state fp32 [{b}, {hv}, {kd}, {vd}], {len(states)} rotating layer states"}


# ---------------------------------------------------------------------------
# model_decode

def bench_model_decode(steps, warmup, cpu, batch=128):
    from yanchor_amd import runtime as rt

    dev = torch.device("cuda:0")
    cfg = rt.ModelConfig()
    model = rt.Model(cfg, batch=batch, device=dev, seed=0)
    _log(f"model_decode: model built, {warmup} warm-up + {steps} timed steps")
    met = rt.run_decode_benchmark(model, steps=steps, warmup=warmup, rate=4.0, prompt_len=128, mean_len=1024,
                                  poll_interval=32)
    _log(f"model_decode: {met.decode_tokens_per_second:.0f} tokens/s; timing the fused GDN decode core")
    roof = gdn_fused_roofline(model)
    res = {
        "value": met.decode_tokens_per_second,
        "unit": "tokens/s",
        "ms_per_step": met.decode_seconds * 1e3 / met.decode_steps,
        "dtype": "bf16",
        "config": {"workload": "model_decode: random-init 4B-shaped hybrid recurrent model (36 layers = 27 GDN "
                               "+ 9 SWA/anchor-memory, hidden 2560, 32 heads, dk=dv=128, 256 anchor slots, "
                               f"vocab 151936), continuous batching over {batch} slots filled before the first step, then "
                               "Poisson(4) arrivals of 128-token prompts, geometric(1024) lengths, refill every "
                               "32 steps, top-k 20 / top-p 0.95 / T 0.6 sampling",
                   "global_batch": batch, "seq_len": 1, "parallelism": "single GPU"},
        "roofline": roof,
        "decode": {"useful_token_events": met.decode_useful_token_events,
                   "scheduled_token_events": met.decode_scheduled_token_events,
                   "decode_seconds": met.decode_seconds, "refill_prefill_seconds": met.refill_prefill_seconds,
                   "wall_seconds": met.generation_wall_seconds, "refilled": met.refilled,
                   "completed": met.completed, "peak_hbm_gib": met.peak_allocated_gib, **met.extra},
    }
    del model
    torch.cuda.empty_cache()
    # beside the line: the reference's throughput profile ("fast": the GDN
    # state stored in float16), the storage of its published batched figures
    _log("model_decode: the same workload with the float16 GDN state")
    model = rt.Model(cfg, batch=batch, device=dev, seed=0, state_dtype=torch.float16)
    m16 = rt.run_decode_benchmark(model, steps=steps, warmup=warmup, rate=4.0, prompt_len=128, mean_len=1024,
                                  poll_interval=32)
    res["fp16_state"] = {"profile": "the reference's 'fast' profile: GDN state stored in float16, updated in "
                                    "float32 (not the headline: the metric's state is float32)",
                         "tokens_per_s": m16.decode_tokens_per_second,
                         "ms_per_step": m16.decode_seconds * 1e3 / m16.decode_steps,
                         "useful_token_events": m16.decode_useful_token_events,
                         "peak_hbm_gib": m16.peak_allocated_gib}
    del model
    torch.cuda.empty_cache()
    _log("model_decode: the chunked prefill and the sampler beside the decode line")
    pre = bench_gdn_prefill(20, 20, False)
    res["prefill"] = {"workload": pre["config"]["workload"], "tokens_per_s": pre["value"],
                      "ms_per_call": pre["roofline"]["avg_launch_us"] * 1e-3, "calls": 20, "warmup_calls": 20,
                      "roofline": pre["roofline"]}
    smp = bench_sampling(100, 20, False, batch=batch)
    res["sampling"] = {"workload": smp["config"]["workload"], "us_per_call": smp["roofline"]["avg_launch_us"],
                       "calls": 100, "roofline": smp["roofline"]}
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = cpu_model_decode(batch)
    return res


def cpu_model_decode(batch, budget_s=20.0, max_steps=32, single_thread=True):
    """Decode steps of the same model shape on the host cores: float32 weights
    (tiled N(0, 0.02) block), every slot live in steady state (positions in
    [1100, 2100): every SWA ring full, every anchor slot committed, the rows
    at staggered points of their commit chunk, so a sixty-fourth of them
    commit at each step), the oracle's recurrence / ring attention / sampler /
    bookkeeping and the batched anchor read and commit of the reference's
    torch branch.  Timed until ``budget_s`` of CPU work (at least one step
    after one warm-up step) on ``cpu_threads()`` threads; then one more step
    on a single thread."""
    from yanchor_amd import runtime as rt
    from yanchor_amd import workloads

    threads = cpu_threads()
    torch.set_num_threads(threads)
    host = cpu_host_info()
    cfg = rt.ModelConfig()
    from oracle.model_ops import BatchedHostOps

    m = rt.Model(cfg, batch=batch, device="cpu", seed=0, ops=BatchedHostOps(), dtype=torch.float32, init="tiled")
    gen = torch.Generator().manual_seed(5)
    tokens = torch.randint(0, cfg.vocab, (batch,), generator=gen)
    positions = torch.randint(1100, 2100, (batch,), generator=gen)
    valid = torch.ones(batch, dtype=torch.bool)
    ids = torch.arange(batch)
    seen = torch.zeros(batch, cfg.vocab, dtype=torch.bool)
    w = cfg.swa_window
    slot = torch.arange(w)
    for i, L in enumerate(m.layers):
        if L["kind"] == "gdn":
            continue
        # the ring holds the last w positions before each row's: slot s the
        # latest p' < p with p' % w == s
        last = (positions - 1)[:, None]
        ring_pos = (last - (last - slot[None]) % w).to(torch.int32)
        m.ring_pos[i].copy_(ring_pos[:, None, :].expand_as(m.ring_pos[i]))
        m.ring_k[i].normal_(generator=gen)
        m.ring_v[i].normal_(generator=gen)
        st = workloads.anchor_state(batch, cfg.kv_heads, cfg.memory_capacity, cfg.memory_chunk, cfg.head_dim,
                                    p_live=1.0, dtype=torch.float32, seed=100 + i)
        st.count.copy_(positions % cfg.memory_chunk)
        st.total.copy_(positions)
        for f in ("keys", "values", "scores", "positions", "pending_keys", "pending_values", "pending_scores",
                  "count", "total"):
            getattr(m.memory[i], f).copy_(getattr(st, f))

    def step(i):
        logits = m.decode_step(tokens, positions + i, valid)
        return m.ops.sample(logits, ids, torch.full((batch,), i + 1), seen, seed=20260923, temperature=0.6,
                            top_k=20, top_p=0.95, penalty=1.5)

    _log("cpu baseline: model built on the host")
    step(0)
    n, t0 = 0, time.perf_counter()
    while True:
        step(n + 1)
        n += 1
        el = time.perf_counter() - t0
        _log(f"cpu baseline: step {n} done, {el:.1f} s")
        if el >= budget_s or n >= max_steps:
            break
    res = {"value": batch * n / el, "unit": "tokens/s", "cores": threads, "kind": "port",
           "sample": f"{n} decode steps x {batch} live slots of the same 36-layer model in float32 on "
                     f"{threads} host threads, steady state (positions 1100-2100: full SWA rings, full anchor "
                     f"memories, staggered commits; every op from the oracle: recurrence, batched anchor read and "
                     f"commit, ring attention, layer glue, sampler), {el:.1f} s; "
                     "refill prefill excluded as in the GPU figure",
           "host": host}
    if single_thread:
        torch.set_num_threads(1)
        t0 = time.perf_counter()
        step(n + 1)
        el1 = time.perf_counter() - t0
        _log(f"cpu baseline: one step on 1 thread, {el1:.1f} s")
        res["single_thread"] = {"value": batch / el1, "unit": "tokens/s", "cores": 1,
                                "sample": f"1 decode step x {batch} live slots on 1 thread, {el1:.1f} s"}
        torch.set_num_threads(threads)
    return res


# ---------------------------------------------------------------------------
# gdn_decode

def bench_gdn_decode(steps, warmup, cpu, batch=64):
    from yanchor_amd import gdn, workloads

    dev = torch.device("cuda:0")
    h, hv, kd, vd, layers = 32, 32, 128, 128, 4
    xs = [workloads.gdn_inputs(batch, 1, h, hv, kd, vd, dtype=torch.bfloat16,
                               seed=workloads.SEED0 + 1 + 1000 * layer, state_std=0.02).to(dev)
          for layer in range(layers)]

    def step(i):
        x = xs[i % layers]
        gdn.recurrent_gated_delta_rule(x.q, x.k, x.v, g=x.g, beta=x.beta, initial_state=x.state)

    ms_per_step, kernel_ms = _time_launches(step, steps, warmup)
    nbytes = gdn_state_bytes(batch, h, hv, kd, vd, 2, 4, False)
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    res = {
        "value": batch / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms_per_step,
        "dtype": "f32",
        "config": {"workload": f"gdn_decode_state_update: one layer decode step, state fp32 "
                               f"[{batch}, 32, 128, 128] in place, bf16 q/k/v, fp32 g/beta, 4 rotating layer states",
                   "global_batch": batch, "seq_len": 1, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": TRAFFIC_GDN_DECODE.get(batch),
                     "kernel": "gdn_recurrent_kernel", "bytes_per_launch": nbytes,
                     "avg_launch_us": kernel_ms * 1e3},
    }
    del xs
    if cpu:
        res["cpu_baseline"] = cpu_gdn_decode(batch, h, hv, kd, vd)
    return res


def bench_long_horizon(steps, warmup, cpu, batch=256, gen_len=32768, prompt_len=256):
    """Long-horizon batched generation: ``batch`` fixed sequences of
    ``gen_len`` tokens from random ``prompt_len``-token prompts on the same
    model with a 16-slot anchor memory committed every 64 tokens (the best 16
    of 80 candidates kept).  Once a sequence is past the 1024-token window
    every ring slot is live (the ring read skips only blocks without a live
    slot) and the 16 memory slots are full, so per-step work no longer depends
    on the position: the default warm-up (800 steps) carries the 256-token
    prompts past the window, and a bounded window of timed steps after it gives
    the sustained rate; the whole horizon would take gen_len steps."""
    from yanchor_amd import runtime as rt

    dev = torch.device("cuda:0")
    cfg = rt.ModelConfig(memory_capacity=16, memory_chunk=64)
    model = rt.Model(cfg, batch=batch, device=dev, seed=0, init="tiled")
    gen = torch.Generator().manual_seed(20260927)
    reqs = [rt.Request(i, torch.randint(0, cfg.vocab, (prompt_len,), generator=gen), gen_len, 0)
            for i in range(batch)]
    _log(f"long_horizon: {batch} sequences x {gen_len} tokens; {warmup} warm-up + {steps} timed steps")
    torch.cuda.reset_peak_memory_stats()
    met = rt.run_decode_benchmark(model, steps=steps, warmup=warmup, poll_interval=1 << 30, requests=reqs,
                                  max_new_tokens=gen_len, progress_every=2048)
    res = {
        "value": met.decode_tokens_per_second,
        "unit": "tokens/s",
        "ms_per_step": met.decode_seconds * 1e3 / met.decode_steps,
        "dtype": "bf16",
        "config": {"workload": f"long_horizon: the 4B-shaped model, {batch} fixed sequences generating {gen_len} "
                               f"tokens from {prompt_len}-token prompts, anchor memory of 16 slots committed every "
                               f"64 tokens; timed over decode steps {warmup + 1}..{warmup + steps} of the horizon",
                   "global_batch": batch, "seq_len": 1, "parallelism": "single GPU"},
        "roofline": gdn_fused_roofline(model),
        "decode": {"useful_token_events": met.decode_useful_token_events, "decode_seconds": met.decode_seconds,
                   "peak_hbm_gib": met.peak_allocated_gib, "positions": [prompt_len + warmup, prompt_len + warmup + steps],
                   "live_slots_end": met.extra.get("live_slots_end")},
    }
    del model
    torch.cuda.empty_cache()
    return res


def bench_gdn_decode_fused(steps, warmup, cpu, batch=128):
    """The fused GDN decode core alone at the model's layer shape, 4 rotating
    layers of synthetic state / conv window / weights."""
    dev = torch.device("cuda:0")
    hv, d, n_layers = 32, 128, 4
    conv_dim = 3 * hv * d
    g = torch.Generator(device=dev).manual_seed(11)

    def rnd(*shape, scale=1.0, dtype=torch.bfloat16):
        return (torch.randn(*shape, device=dev, generator=g) * scale).to(dtype)

    layers_in = [(rnd(batch, 3, conv_dim), rnd(conv_dim, 4, scale=0.5),
                  torch.log(torch.linspace(1.0, 16.0, hv, device=dev)), torch.linspace(-1.0, 1.0, hv, device=dev),
                  rnd(batch, hv, d, d, scale=0.02, dtype=torch.float32), rnd(d, scale=0.1))
                 for _ in range(n_layers)]
    step = _fused_step(dev, batch, hv, d, conv_dim, layers_in, seed=12)
    ms_per_step, kernel_ms = _time_launches(step, steps, warmup)
    nbytes = gdn_fused_bytes(batch, hv, d, conv_dim)
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    res = {
        "value": batch / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms_per_step,
        "dtype": "f32",
        "config": {"workload": f"gdn_decode_fused: one GDN layer's decode core (conv update, state update, "
                               f"gated norm), state fp32 [{batch}, 32, 128, 128] in place, bf16 projection row, "
                               f"4 rotating layers", "global_batch": batch, "seq_len": 1,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": TRAFFIC_GDN_FUSED.get(batch),
                     "kernel": "gdn_decode_fused_kernel", "bytes_per_launch": nbytes,
                     "avg_launch_us": kernel_ms * 1e3},
    }
    if cpu:
        res["cpu_baseline"] = cpu_gdn_decode(batch, 32, hv, d, d)
    return res


def cpu_gdn_decode(b, h, hv, kd, vd, budget_s=12.0) -> dict:
    """The oracle's token recurrence in torch float32 on the host cores, on the
    same decode shape, repeated until ~budget_s of CPU work."""
    from oracle import gdn as ref
    from yanchor_amd import workloads

    threads = cpu_threads()
    torch.set_num_threads(threads)
    x = workloads.gdn_inputs(b, 1, h, hv, kd, vd, dtype=torch.bfloat16, seed=workloads.SEED0 + 1, state_std=0.02)
    state = x.state
    ref.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, state, dtype=torch.float32)
    n, t0 = 0, time.perf_counter()
    while True:
        _, state = ref.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, state, dtype=torch.float32)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 2000:
            break
    return {"value": b * n / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode steps of the same layer shape (B={b}, HV={hv}, dk=dv={kd}) with the "
                      f"float32 torch oracle, {el:.1f} s"}


CHUNK = 64
MFMA_BF16_PEAK_TFLOPS = 2500.0


def chunk_flops(n_chunks, heads, d=128, c=CHUNK):
    """Algorithmic FLOP of the chunked form: per (chunk, head)
    10 C^2 d + 6 C d^2 + 2/3 C^3 (the intra-chunk products, the WY/UT
    transform and the state scan)."""
    return n_chunks * heads * (10 * c * c * d + 6 * c * d * d + (2 * c ** 3) / 3)


def bench_gdn_prefill(steps, warmup, cpu, batch=None):
    """Varlen chunked prefill of one GDN layer: 32 packed sequences with
    lengths uniform in [512, 8192] (seeded), H = HV = 32, dk = dv = 128, bf16
    q/k/v/o, fp32 gates and final states, zero initial state."""
    from yanchor_amd import gdn, workloads

    del batch
    lengths = workloads.prefill_lengths()
    h = hv = 32
    d = 128
    x = workloads.packed_inputs(lengths, h, hv, d, d).to("cuda:0")

    def step(i):
        gdn.chunk_gated_delta_rule(x.q, x.k, x.v, g=x.g, beta=x.beta, output_final_state=True,
                                   use_qk_l2norm_in_kernel=True, cu_seqlens=x.cu_seqlens, lengths=lengths)

    ms_per_step, kernel_ms = _time_launches(step, steps, warmup)
    tokens = sum(lengths)
    n_chunks = sum(-(-n // CHUNK) for n in lengths)
    flops = chunk_flops(n_chunks, hv, d)
    nbytes = tokens * (h * d * 2 * 2 + hv * d * 2 * 2 + hv * 8) + len(lengths) * hv * d * d * 4
    gbs = nbytes / (kernel_ms * 1e-3) / 1e9
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    res = {"metric": "varlen chunked prefill tokens/s, one GDN layer (MFMA utilisation and HBM fraction)",
           "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s", "ms_per_step": ms_per_step, "dtype": "bf16",
           "config": {"workload": f"gdn_prefill: {len(lengths)} packed sequences, lengths U[512, 8192] "
                                  f"({tokens} tokens), H=HV=32, dk=dv=128, chunk 64, bf16 q/k/v/o, fp32 gates/state",
                      "global_batch": len(lengths), "seq_len": tokens, "parallelism": "single GPU"},
           "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": gbs / HBM_PEAK_GBS, "traffic": TRAFFIC_PREFILL,
                        "traffic_source": TRAFFIC_SOURCE, "kernel": "chunk_fused_kernel",
                        "bytes_per_launch": nbytes, "avg_launch_us": kernel_ms * 1e3,
                        "mfma_tflops": tflops, "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                        "mfma_util": tflops / MFMA_BF16_PEAK_TFLOPS, "flops_per_launch": flops,
                        "roofline_frac": max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (MFMA_BF16_PEAK_TFLOPS * 1e12))
                        / (kernel_ms * 1e-3)}}
    del x
    if cpu:
        res["cpu_baseline"] = cpu_gdn_prefill(lengths, h, hv, d)
    return res


def cpu_gdn_prefill(lengths, h, hv, d, budget_s=15.0):
    """The oracle's chunked form in float32 on the host cores, sequence by
    sequence over the same packed set until ~budget_s."""
    from oracle import gdn as ref
    from yanchor_amd import workloads

    threads = cpu_threads()
    torch.set_num_threads(threads)
    x = workloads.packed_inputs(lengths, h, hv, d, d)
    cu = x.cu_seqlens.tolist()
    n_tok, n_seq, t0 = 0, 0, time.perf_counter()
    for i in range(len(lengths)):
        sl = slice(cu[i], cu[i + 1])
        ref.chunk_gated_delta_rule(x.q[:, sl], x.k[:, sl], x.v[:, sl], x.g[:, sl], x.beta[:, sl],
                                   dtype=torch.float32)
        n_tok += lengths[i]
        n_seq += 1
        el = time.perf_counter() - t0
        _log(f"cpu baseline: sequence {n_seq} ({lengths[i]} tokens) done, {el:.1f} s")
        if el >= budget_s:
            break
    return {"value": n_tok / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the first {n_seq} of the same packed sequences ({n_tok} tokens, all 32 heads) through "
                      f"the float32 torch oracle's chunked form, {el:.1f} s"}


def bench_anchor_read(steps, warmup, cpu, batch=64):
    """Anchor-memory read of one decode token (committed_gqa) at the decode
    config: 64 rows, 32 heads with a memory per head, 256 slots of 128 bf16
    dims, each slot live with p = 0.7; three rotating states (806 MB) so the
    slots stream from HBM."""
    from yanchor_amd import independent_memory as im, workloads

    del cpu
    g, cap, d, n_states = 32, 256, 128, 3
    states = [workloads.anchor_state(batch, g, cap, 64, d, seed=workloads.SEED0 + 1 + 7 * i)
              for i in range(n_states)]
    for st in states:
        st.to_("cuda:0")
    q = workloads.anchor_query(batch, g, d).to("cuda:0")

    def step(i):
        im.committed_gqa(q, states[i % n_states])

    ms_per_step, kernel_ms = _time_launches(step, steps, warmup)
    # algorithmic bytes: the key and value rows of the live slots (a dead
    # slot's row enters neither the softmax nor the sum), every position, the
    # query and the output; the mean over the rotating states
    live = sum(int((st.positions >= 0).sum()) for st in states) / n_states
    nbytes = int(2 * live * d * 2) + batch * g * cap * 4 + 2 * batch * g * d * 2
    dense = 2 * batch * g * cap * d * 2 + batch * g * cap * 4 + 2 * batch * g * d * 2
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    del states
    return {"metric": "anchor-memory read per decode token (HBM GB/s)", "value": achieved, "unit": "GB/s",
            "ms_per_step": ms_per_step, "dtype": "bf16",
            "config": {"workload": f"anchor_read: committed_gqa, {batch} rows x {g} heads x {cap} slots x {d} "
                                   "bf16, p_live 0.7, 3 rotating states", "global_batch": batch, "seq_len": 1,
                       "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": TRAFFIC_ANCHOR_READ if batch == 64 else None,
                         "traffic_source": TRAFFIC_SOURCE if batch == 64 else None, "kernel": "anchor_read_kernel",
                         "bytes_per_launch": nbytes, "live_slot_fraction": live / (batch * g * cap),
                         "dense_bytes_per_launch": dense, "avg_launch_us": kernel_ms * 1e3}}


def hbm_stream_rates(steps, warmup, gib=1, grid=16384):
    """GB/s of the library's calibration streams (yh_hbm_stream) over two
    `gib` GiB buffers: copy, in-place read-modify-write, read and write, each
    with plain and with nontemporal loads and stores -- what a streaming
    kernel reaches on this GPU, beside the 8 TB/s spec figure."""
    from yanchor_amd import _native

    nbytes = gib << 30
    a = torch.zeros(nbytes // 4, device="cuda:0")
    b = torch.zeros_like(a)
    st = torch.cuda.current_stream().cuda_stream
    rates = {}
    for kind, name, moved in ((0, "copy", 2 * nbytes), (1, "rmw", 2 * nbytes), (2, "read", nbytes),
                              (3, "write", nbytes)):
        for nt in (0, 1):
            def step(i, kind=kind, nt=nt):
                _native.call("yh_hbm_stream", kind, nt, a.data_ptr(), b.data_ptr(), nbytes, grid, st)
            _, ms = _time_launches(step, steps, warmup)
            rates[f"{name}{'_nt' if nt else ''}"] = round(moved / (ms * 1e-3) / 1e9, 1)
    del a, b
    return rates


def bench_anchor_prefill(steps, warmup, cpu, batch=32):
    """The anchor-memory half of a prefill that continues a state
    (independent_memory.sequence: the prefix Top-K scan, the MFMA read of
    every C-token block over the memory committed before it, the commit) for
    B rows of 2048 tokens, 32 heads over 8 memories of 256 slots, C = 64,
    bf16; and the block read (yh_indexed_gqa) alone on the same shapes for its
    roofline."""
    from yanchor_amd import independent_memory as im, workloads

    del cpu
    b, length, h, g, cap, c, d = batch, 2048, 32, 8, 256, 64, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(20260928)
    state = workloads.anchor_state(b, g, cap, c, d, p_live=0.9, seed=workloads.SEED0 + 11)
    state.to_("cuda:0")
    q = torch.randn(b, length, h, d, generator=gen).to(torch.bfloat16).to(dev)
    k = torch.randn(b, length, g, d, generator=gen).to(torch.bfloat16).to(dev)
    v = torch.randn(b, length, g, d, generator=gen).to(torch.bfloat16).to(dev)
    sc = torch.randn(b, length, g, generator=gen).to(dev)

    def step(i):
        im.sequence(q, k, v, sc, None, c, state)

    ms_per_step, kernel_ms = _time_launches(step, steps, warmup)
    # the block read alone: every block of every row reads cap referenced rows
    # of its group among the sources (committed slots, pending slots, tokens)
    blocks = length // c + 1
    n_src = cap + c + length
    qb = torch.randn(b, blocks, c, h, d, generator=gen).to(torch.bfloat16).to(dev)
    src_k = torch.randn(b, n_src, g, d, generator=gen).to(torch.bfloat16).to(dev)
    src_v = torch.randn(b, n_src, g, d, generator=gen).to(torch.bfloat16).to(dev)
    refs = torch.randint(0, n_src, (b, blocks, g, cap), generator=gen, dtype=torch.int32).to(dev)
    _, read_ms = _time_launches(lambda i: im.indexed_gqa(qb, src_k, src_v, refs), steps, warmup)
    flops = 4.0 * b * blocks * h * c * cap * d           # Q K^T and P V over the referenced rows
    nbytes = 2 * qb.numel() * 2 + 2 * src_k.numel() * 2 + refs.numel() * 4   # q and out, the sources once, refs
    t_hbm, t_mfma = nbytes / (HBM_PEAK_GBS * 1e9), flops / 2.5e15
    achieved = nbytes / (read_ms * 1e-3) / 1e9
    return {"metric": "anchor-memory prefill tokens/s (sequence with a state)",
            "value": b * length / (kernel_ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms_per_step,
            "dtype": "bf16",
            "config": {"workload": f"anchor_prefill: {b} rows x {length} tokens, {h} heads over {g} memories of "
                                   f"{cap} slots x {d} bf16, chunk {c}, continuing a state (p_live 0.9)",
                       "global_batch": b, "seq_len": length, "parallelism": "single GPU"},
            "roofline": {"bound": "hbm" if t_hbm >= t_mfma else "mfma", "achieved": achieved,
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": max(t_hbm, t_mfma) / (read_ms * 1e-3),
                         "traffic": None, "kernel": "indexed_gqa_kernel", "bytes_per_launch": nbytes,
                         "flops_per_launch": flops, "mfma_tflops": flops / (read_ms * 1e-3) / 1e12,
                         "avg_launch_us": read_ms * 1e3, "sequence_call_us": kernel_ms * 1e3}}


def bench_sampling(steps, warmup, cpu, batch=128):
    """The decode step's sampler (top-k 20 / top-p 0.95 / T 0.6, the fused
    top-20 semantics, presence penalty 1.5 fused in) on B rows of bf16 logits
    over the 151936-token vocabulary; six rotating (logits, seen) sets, 350 MB,
    so the rows stream from HBM."""
    from yanchor_amd import inference_kernels as ik

    del cpu
    v, n_sets = 151936, 6
    gen = torch.Generator().manual_seed(20260927)
    sets = []
    for _ in range(n_sets):
        logits = (torch.randn(batch, v, generator=gen) * 2.0).to(torch.bfloat16).to("cuda:0")
        seen = (torch.rand(batch, v, generator=gen) < 0.007).to("cuda:0")
        sets.append((logits, seen))
    ids = torch.arange(batch, dtype=torch.int64, device="cuda:0")

    def step(i):
        logits, seen = sets[i % n_sets]
        ik.topk_sample(logits, ids, i, seed=7, temperature=0.6, top_k=20, top_p=0.95, mode=ik.SAMPLE_FUSED,
                       seen=seen, presence_penalty=1.5)

    ms_per_step, kernel_ms = _time_launches(step, steps, warmup)
    # algorithmic bytes: every bf16 logit and every byte of the seen mask, the
    # ids and the tokens
    nbytes = batch * v * 2 + batch * v + 2 * batch * 8
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    return {"metric": "top-k / top-p sampling of one decode step (HBM GB/s)", "value": achieved, "unit": "GB/s",
            "ms_per_step": ms_per_step, "dtype": "bf16",
            "config": {"workload": f"sampling: {batch} rows x {v} bf16 logits, presence mask, top-k 20, top-p 0.95, "
                                   "T 0.6, penalty 1.5, 6 rotating sets", "global_batch": batch, "seq_len": 1,
                       "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "topk_wide_kernel + "
                         "sample_rows_kernel", "bytes_per_launch": nbytes, "avg_launch_us": kernel_ms * 1e3}}


# The decode step's projections at the 4B shape: (name, N, K, epilogue), the
# packed weights' shapes per layer (GDN: input and output; attention: q/k/v
# and output; anchor memory: fused input, fused k/v ([u | act] against
# [W_kv | W_kv W_down]), output; MLP: gate/up with the silu epilogue and down;
# lm_head) with their calls per step.
DECODE_PROJECTIONS = [("mlp_gate_up", 19456, 2560, "silu", 36), ("mlp_down", 2560, 9728, "defer", 36),
                      ("gdn_in", 16448, 2560, "", 27), ("gdn_out", 2560, 4096, "defer", 27),
                      ("attn_qkv", 10240, 2560, "", 9), ("attn_o", 2560, 4096, "", 9),
                      ("memory_in", 9280, 2560, "", 9), ("memory_kv_fused", 2048, 5120, "", 9),
                      ("memory_o", 2560, 4096, "defer", 9),
                      ("lm_head", 151936, 2560, "", 1)]


def bench_projections(steps, warmup, cpu, batch=128):
    """Every decode projection of the 4B-shaped model at M = batch rows on
    the packed-weight kernels, as the decode step calls them (silu
    epilogue; split-K partials left to the next norm where the step defers
    them; the residual add), each in a HIP graph of 32 calls over rotating
    weight copies (> 600 MB, past the Infinity Cache), beside hipBLASLt on the
    row-major weights.  value = weight bytes of one decode step's
    projections / their summed time."""
    from yanchor_amd import _native, layers

    del cpu
    dev = torch.device("cuda:0")
    calls = 32
    out = {}
    step_bytes = step_us = blas_us = 0.0

    def graph_us(fn, reps=max(2, steps // 32)):
        for i in range(max(1, warmup // 32)):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(calls):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * calls)

    for name, n, k, epi, per_step in DECODE_PROJECTIONS:
        copies = max(2, math.ceil(600e6 / (n * k * 2)))
        gen = torch.Generator(device=dev).manual_seed(7)
        ws = [(torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16) for _ in range(copies)]
        pws = [layers.PackedWeight(w, pair_halves=epi == "silu") for w in ws]
        x = torch.randn(batch, k, device=dev, generator=gen).to(torch.bfloat16)
        res = torch.randn(batch, n, device=dev, generator=gen).to(torch.bfloat16) if epi == "residual" else None
        if epi == "silu":
            fn = lambda i: layers.linear_silu(x, pws[i % copies])  # noqa: E731
        else:
            fn = lambda i: layers.linear(x, pws[i % copies], residual=res, defer=epi == "defer")  # noqa: E731
        us = graph_us(fn)
        ref = graph_us(lambda i: torch.matmul(x, ws[i % copies].t()))
        nbytes = n * k * 2
        split = 1 if epi == "silu" else int(_native.lib().yh_linear_packed_split(batch, n, k))
        out[name] = {"shape": [batch, n, k], "epilogue": epi or "plain", "split_k": split, "us": round(us, 2),
                     "tb_s": round(nbytes / us / 1e6, 3), "hipblaslt_us": round(ref, 2), "calls_per_step": per_step}
        _log(f"projections: {name} {n}x{k}: {us:.1f} us ({nbytes / us / 1e6:.2f} TB/s), hipBLASLt {ref:.1f} us")
        step_bytes += per_step * nbytes
        step_us += per_step * us
        blas_us += per_step * ref
        del ws, pws
        torch.cuda.empty_cache()
    achieved = step_bytes / step_us / 1e3
    return {"metric": "decode-step projections at M=128: weight bytes / summed kernel time (HBM GB/s)",
            "value": achieved, "unit": "GB/s", "ms_per_step": step_us * 1e-3, "dtype": "bf16",
            "config": {"workload": f"projections: the 4B-shaped model's decode projections at M={batch} "
                                   "(packed weights, graphs of 32 calls over rotating weights)",
                       "global_batch": batch, "seq_len": 1, "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "proj_kernel",
                         "bytes_per_launch": step_bytes, "avg_launch_us": step_us},
            "projections": out, "hipblaslt_ms_per_step": blas_us * 1e-3}


def bench_hbm_copy(steps, warmup, cpu, batch=None):
    """A plain 128 MiB device-to-device copy (torch's copy kernel): the
    calibration kernel for the HBM byte counters; beside it the rates of the
    library's calibration streams over 1 GiB buffers."""
    del cpu, batch
    n = 32 << 20
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    ms_per_step, kernel_ms = _time_launches(lambda i: dst.copy_(src), steps, warmup)
    nbytes = 2 * n * 4
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    del src, dst
    streams = hbm_stream_rates(steps, warmup)
    # the dense bf16 MFMA rate a large library GEMM reaches (8192^3 on hipBLASLt)
    n = 8192
    ga = torch.randn(n, n, device="cuda:0").to(torch.bfloat16)
    gb = torch.randn(n, n, device="cuda:0").to(torch.bfloat16)
    gc = torch.empty(n, n, device="cuda:0", dtype=torch.bfloat16)
    _, gemm_ms = _time_launches(lambda i: torch.matmul(ga, gb, out=gc), steps, warmup)
    gemm_tflops = 2.0 * n ** 3 / (gemm_ms * 1e-3) / 1e12
    del ga, gb, gc
    return {"metric": "device copy bandwidth (HBM GB/s)", "value": achieved, "unit": "GB/s",
            "ms_per_step": ms_per_step, "dtype": "f32",
            "config": {"workload": "hbm_copy: 128 MiB float32 device copy (read 128 MiB + write 128 MiB)",
                       "global_batch": 1, "seq_len": 1, "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "copy",
                         "bytes_per_launch": nbytes, "avg_launch_us": kernel_ms * 1e3},
            "hbm_streams_gbs": {"buffers": "two 1 GiB float32 buffers, 16384 workgroups of 256 threads",
                                **streams},
            "gemm_bf16": {"shape": "8192 x 8192 x 8192 torch.matmul (hipBLASLt)", "tflops": round(gemm_tflops, 1),
                          "frac_of_2500": round(gemm_tflops / 2500.0, 3)}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (model_decode 2048, gdn_decode 200)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (model_decode 64, gdn_decode 20)")
    ap.add_argument("--workload", default="model_decode",
                    choices=["model_decode", "long_horizon", "gdn_decode", "gdn_decode_fused", "gdn_prefill",
                             "anchor_read", "anchor_prefill", "sampling", "projections", "hbm_copy"])
    ap.add_argument("--batch", type=int, default=None, help="slots (model_decode 128) / rows (gdn_decode 64)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: every run here has one "
              "GPU (the decode path shards by sequence slot with no exchange between GPUs)", file=sys.stderr)
        return 2
    if args.workload == "model_decode":
        steps, warmup = args.steps or 2048, 64 if args.warmup is None else args.warmup
        res = bench_model_decode(steps, warmup, not args.no_cpu, batch=args.batch or 128)
    elif args.workload == "long_horizon":
        steps, warmup = args.steps or 512, 800 if args.warmup is None else args.warmup
        res = bench_long_horizon(steps, warmup, not args.no_cpu, batch=args.batch or 256)
    else:
        steps, warmup = args.steps or 200, 20 if args.warmup is None else args.warmup
        fn = {"gdn_decode": bench_gdn_decode, "gdn_decode_fused": bench_gdn_decode_fused,
              "gdn_prefill": bench_gdn_prefill, "anchor_read": bench_anchor_read, "sampling": bench_sampling,
              "anchor_prefill": bench_anchor_prefill, "projections": bench_projections,
              "hbm_copy": bench_hbm_copy}
        res = fn[args.workload](steps, warmup, not args.no_cpu,
                                batch=args.batch or (128 if args.workload in ("gdn_decode_fused", "sampling",
                                                                              "projections") else
                                                     32 if args.workload == "anchor_prefill" else 64))
    line = {"metric": res.get("metric", METRIC), "value": res["value"], "unit": res["unit"], "n_gpus": 1,
            "steps": steps, "warmup": warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": res["dtype"], "data": "synthetic (seeded random-init weights and requests)",
            "config": res["config"], "roofline": res["roofline"]}
    for key in ("cpu_baseline", "decode", "fp16_state", "prefill", "sampling", "projections", "hipblaslt_ms_per_step",
                "hbm_streams_gbs", "gemm_bf16"):
        if key in res:
            line[key] = res[key]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
