"""Write tests/golden/counter_sampling.npz from the reference's own functions.

The counter hash and the torch sampler have no closed form or library routine
that pins them, so their vectors come from the reference implementation itself:
runtime/model/inference_kernels.py (counter_uniform 24-33,
top_k_top_p_distribution 42-58, sample_top_k_top_p_counter 73-88).  Run in the
development container only (it reads /root/reference); the .npz it writes is
the committed fixture.

    python tests/golden/make_counter_sampling.py
"""
import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

sys.dont_write_bytecode = True  # never write into the read-only reference tree
REF = Path("/root/reference/runtime/model/inference_kernels.py")
OUT = Path(__file__).resolve().parent / "counter_sampling.npz"


def main():
    spec = importlib.util.spec_from_file_location("ref_inference_kernels", REF)
    ref = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = ref
    spec.loader.exec_module(ref)

    gen = torch.Generator().manual_seed(20260923)
    ids = torch.cat([torch.arange(0, 40), torch.randint(0, 2**40, (24,), generator=gen)]).long()
    steps = torch.cat([torch.arange(0, 40), torch.randint(0, 2**33, (24,), generator=gen)]).long()
    rows = {}
    for seed, stream in ((20260923, 0), (20260820, 0), (7, 3), (2**32 + 11, 2**32 + 5)):
        u = ref.counter_uniform(ids, steps, seed=seed, stream=stream, dtype=torch.float32)
        rows[f"uniform_{seed}_{stream}"] = u.numpy()
    out = {"ids": ids.numpy(), "steps": steps.numpy()}
    out.update(rows)
    out["uniform_keys"] = np.array([f"{s}_{t}" for s, t in ((20260923, 0), (20260820, 0), (7, 3),
                                                            (2**32 + 11, 2**32 + 5))])

    # the torch sampler on seeded logits
    b, v = 16, 512
    logits = (torch.randn(b, v, generator=gen) * 3.0).float()
    att = torch.randint(0, 10**6, (b,), generator=gen).long()
    st = torch.randint(0, 5000, (b,), generator=gen).long()
    out["logits"] = logits.numpy()
    out["attempt_ids"] = att.numpy()
    out["row_steps"] = st.numpy()
    cases = [(0.6, 20, 0.95, 20260923), (1.0, 20, 0.95, 20260923), (0.6, 20, 1.0, 5), (1.3, 7, 0.5, 99),
             (0.6, 1, 0.95, 1), (0.8, 64, 0.9, 123)]
    out["sample_cases"] = np.array(cases, dtype=np.float64)
    for i, (t, k, p, seed) in enumerate(cases):
        tok = ref.sample_top_k_top_p_counter(logits, att, st, seed=int(seed), temperature=t, top_k=int(k),
                                             top_p=p)
        out[f"tokens_{i}"] = tok.numpy()
        if int(k) > 1:
            idx, probs = ref.top_k_top_p_distribution(logits, temperature=t, top_k=int(k), top_p=p)
            out[f"dist_idx_{i}"] = idx.numpy()
            out[f"dist_p_{i}"] = probs.numpy()
    # the full-vocabulary branches (inference_kernels.py:78-86): top_k <= 0
    # with top_p == 1 (vocabulary order), top_k <= 0 with top_p < 1 and
    # top_k > 64 (value order, truncated at top_p); on the same logits and
    # on bf16-valued logits (exact ties)
    full_cases = [(0.6, 0, 1.0, 20260923), (1.0, -1, 1.0, 7), (0.8, 0, 0.9, 123), (0.7, 100, 0.95, 5),
                  (1.3, 300, 1.0, 11), (0.6, 0, 0.5, 77), (2.0, 65, 0.99, 3)]
    out["full_cases"] = np.array(full_cases, dtype=np.float64)
    logits_bf16 = (torch.randn(b, v, generator=gen) * 3.0).to(torch.bfloat16).float()
    out["logits_bf16"] = logits_bf16.numpy()
    for name, lg in (("", logits), ("bf16_", logits_bf16)):
        for i, (t, k, p, seed) in enumerate(full_cases):
            tok = ref.sample_top_k_top_p_counter(lg, att, st, seed=int(seed), temperature=t, top_k=int(k), top_p=p)
            out[f"full_{name}tokens_{i}"] = tok.numpy()
    np.savez(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
