"""yh_topk_sample_noalloc (the sampler with its scratch in a static device
array) against yh_topk_sample with a caller-owned workspace, through the C ABI
(GPU).

Two calls in a row, the second with a smaller input, in both sampling
semantics: the tokens and the returned top-k values and indices must be equal
bit for bit.  A size past the static maximum is refused before any launch.
"""

import pytest
import torch

from yanchor_amd import _native as N
from yanchor_amd import inference_kernels as ik

pytestmark = pytest.mark.gpu

STATIC_BYTES = 8 << 20


def _args(b, v, k, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    scores = torch.randn(b, v, device=dev, generator=g).to(torch.bfloat16)
    seen = torch.rand(b, v, device=dev, generator=g) < 0.01
    ids = torch.arange(1000, 1000 + b, device=dev, dtype=torch.int64)
    steps = torch.randint(0, 500, (b,), device=dev, generator=g, dtype=torch.int64)
    return scores, seen, ids, steps


def _run(noalloc, scores, seen, ids, steps, k, mode, penalty):
    b, v = scores.shape
    dev = scores.device
    tokens = torch.full((b, 1), -1, dtype=torch.int64, device=dev)
    vals = torch.full((b, k), float("nan"), dtype=torch.float32, device=dev)
    idxs = torch.full((b, k), -1, dtype=torch.int64, device=dev)
    common = (scores.data_ptr(), N.code(scores), scores.stride(0), seen.data_ptr(), seen.stride(0), float(penalty),
              ids.data_ptr(), steps.data_ptr(), 0, 20260923, 0, 0.6, k, 0.95, mode, tokens.data_ptr(),
              vals.data_ptr(), idxs.data_ptr())
    if noalloc:
        N.call("yh_topk_sample_noalloc", *common, b, v, N.stream_of(scores))
    else:
        ws = torch.empty(int(N.lib().yh_topk_workspace_bytes(b, v, k)), dtype=torch.uint8, device=dev)
        N.call("yh_topk_sample", *common, ws.data_ptr(), ws.numel(), b, v, N.stream_of(scores))
    torch.cuda.synchronize()
    return tokens.cpu(), vals.cpu(), idxs.cpu()


@pytest.mark.parametrize("mode,k,penalty", [(ik.SAMPLE_FUSED, 20, 1.5), (ik.SAMPLE_TORCH, 64, 0.0)],
                         ids=["fused_top20_penalty", "torch_top64"])
def test_noalloc_matches_workspace_sampler(gpu, mode, k, penalty):
    # the decode batch at the full vocabulary, then a smaller one: the second
    # call reuses the scratch the first one filled
    for b, v, seed in ((128, 151936, 1), (5, 40000, 2)):
        print(f"noalloc sampler: B={b} V={v} k={k} mode={mode}", flush=True)
        assert N.lib().yh_topk_workspace_bytes(b, v, k) <= STATIC_BYTES
        args = _args(b, v, k, seed, gpu)
        want = _run(False, *args, k, mode, penalty)
        got = _run(True, *args, k, mode, penalty)
        assert int(want[0].min()) >= 0
        for x, y in zip(got, want):
            assert torch.equal(x, y)


def test_noalloc_refuses_sizes_past_the_static_maximum(gpu):
    b, v, k = 1024, 151936, 64          # 1024 x 19 x 64 x 8 bytes > 8 MiB
    assert N.lib().yh_topk_workspace_bytes(b, v, k) > STATIC_BYTES
    scores = torch.empty(1, 1, device=gpu)
    with pytest.raises(N.NativeError, match="static maximum"):
        N.call("yh_topk_sample_noalloc", scores.data_ptr(), N.F32, v, None, 0, 0.0, scores.data_ptr(), None, 0,
               1, 0, 1.0, k, 1.0, ik.SAMPLE_TORCH, scores.data_ptr(), None, None, b, v, N.stream_of(scores))
