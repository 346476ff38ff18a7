"""Benchmark of the YANchor recurrent decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints one JSON line.  Workloads:

* ``gdn_decode`` (default): one decode step of the gated-delta state update on
  the decode configuration -- 64 live sequences, HV = 32 heads,
  dk = dv = 128, fp32 state [64, 32, 128, 128] ~ N(0, 0.02) updated in place,
  bf16 q/k/v, fp32 g/beta.  Steps cycle over 4 independent layer states
  (4 x 128 MiB) so no launch finds its state in the 256 MB Infinity Cache
  left behind by the previous one.  value = decode tokens/s of that layer step
  (64 tokens per step).  The same step through a 96-row slot pool with
  state_indices (the vLLM-style indirection) is reported as ``pooled_slots``.

Timing: W untimed steps, then K steps between two stream synchronisations,
with HIP events (torch.cuda.Event on the stream the kernels are launched on)
around the timed region.  ``roofline`` prices the state-update kernel's
algorithmic bytes per launch against the 8 TB/s HBM peak.  ``cpu_baseline``
times the CPU oracle (torch float32, host threads) on a bounded sample of the
same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of gdn_recurrent_kernel on the decode workload, from
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (KiB per dispatch) scaled by the same
# counters on a copy kernel of known size (FETCH x 2.0, WRITE x 1.0).
TRAFFIC_GDN_DECODE = None
METRIC = "decode tokens/s at B=128 on 1 GPU; state-update HBM GB/s as % of peak"


def gdn_state_bytes(b, h, hv, kd, vd, qkv_size, gate_size, with_indices):
    """Algorithmic HBM bytes of one decode step of the state update."""
    state = 2 * b * hv * kd * vd * 4            # fp32 state read + write
    inputs = b * (2 * h * kd + hv * vd) * qkv_size  # q, k, v
    gates = 2 * b * hv * gate_size                # g, beta
    out = b * hv * vd * qkv_size                  # o
    idx = 4 * b if with_indices else 0
    return state + inputs + gates + out + idx


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _time_steps(step, steps, warmup):
    """W untimed steps, then K timed steps between stream synchronisations.
    Returns (wall ms per step, event ms per step on the launch stream)."""
    import torch
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


def bench_gdn_decode(steps: int, warmup: int, cpu: bool) -> dict:
    """Decode state update on the [64, 32, 128, 128] fp32 state (rows indexed
    densely, like the reference's in-place decode launch), plus the same step
    through a 96-slot pool with state_indices as a secondary figure."""
    import torch
    from yanchor_amd import gdn, workloads

    dev = torch.device("cuda:0")
    b, h, hv, kd, vd, layers = 64, 32, 32, 128, 128, 4

    def make(pool):
        xs = []
        for layer in range(layers):
            x = workloads.gdn_inputs(b, 1, h, hv, kd, vd, dtype=torch.bfloat16,
                                     seed=workloads.SEED0 + 1 + 1000 * layer, state_std=0.02,
                                     pool_rows=pool).to(dev)
            if pool is None:
                x.state_indices = None
            xs.append(x)
        return xs

    def stepper(xs):
        def step(i):
            x = xs[i % layers]
            gdn.recurrent_gated_delta_rule(x.q, x.k, x.v, g=x.g, beta=x.beta,
                                           initial_state=x.state, state_indices=x.state_indices)
        return step

    xs = make(None)
    torch.cuda.synchronize()
    ms_per_step, kernel_ms = _time_steps(stepper(xs), steps, warmup)
    del xs
    pooled = make(96)
    _, pooled_ms = _time_steps(stepper(pooled), steps, warmup)
    del pooled
    torch.cuda.empty_cache()
    nbytes = gdn_state_bytes(b, h, hv, kd, vd, 2, 4, False)
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    pooled_gbs = gdn_state_bytes(b, h, hv, kd, vd, 2, 4, True) / (pooled_ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": b / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms_per_step,
        "dtype": "f32",
        "config": {"workload": "gdn_decode_state_update: one layer decode step, state fp32 "
                               "[64, 32, 128, 128] in place, bf16 q/k/v, fp32 g/beta, "
                               "4 rotating layer states",
                   "global_batch": b, "seq_len": 1, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": TRAFFIC_GDN_DECODE,
                     "kernel": "gdn_recurrent_kernel", "bytes_per_launch": nbytes,
                     "avg_launch_us": kernel_ms * 1e3},
        "pooled_slots": {"pool_rows": 96, "avg_launch_us": pooled_ms * 1e3,
                         "achieved_GBs": pooled_gbs, "frac": pooled_gbs / HBM_PEAK_GBS},
    }
    if cpu:
        res["cpu_baseline"] = cpu_gdn_decode(b, h, hv, kd, vd)
    return res


def cpu_gdn_decode(b, h, hv, kd, vd, budget_s=12.0) -> dict:
    """The oracle's token recurrence in torch float32 on the host cores, on the
    same decode shape, repeated until ~budget_s of CPU work."""
    import torch
    from oracle import gdn as ref
    from yanchor_amd import workloads

    threads = cpu_threads()
    torch.set_num_threads(threads)
    x = workloads.gdn_inputs(b, 1, h, hv, kd, vd, dtype=torch.bfloat16, seed=workloads.SEED0 + 1,
                             state_std=0.02)
    state = x.state
    for _ in range(2):
        ref.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, state, dtype=torch.float32)
    n, t0 = 0, time.perf_counter()
    while True:
        _, state = ref.recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, state,
                                                  dtype=torch.float32)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 2000:
            break
    return {"value": b * n / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode steps of the same layer shape (B={b}, HV={hv}, "
                      f"dk=dv={kd}) with the float32 torch oracle, {el:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="gdn_decode", choices=["gdn_decode"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the hot path shards by sequence with no exchange; see the design notes)",
              file=sys.stderr)
        return 2
    res = bench_gdn_decode(args.steps, args.warmup, not args.no_cpu)
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": res["dtype"], "data": "synthetic (seeded torch.Generator)",
            "config": res["config"], "roofline": res["roofline"]}
    if "cpu_baseline" in res:
        line["cpu_baseline"] = res["cpu_baseline"]
    if "pooled_slots" in res:
        line["pooled_slots"] = res["pooled_slots"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
