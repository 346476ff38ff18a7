"""The C-ABI library loads and exports every entry point include/*.h declares.

Runs without a GPU: it only resolves symbols and checks argument validation
paths that return before any device work.
"""
import ctypes
import re
from pathlib import Path

import pytest

from yanchor_amd import _native

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(yh_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "yh_gdn_recurrent" in names and "yh_last_error" in names


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        pytest.fail(f"native library not built at {_native.LIB_PATH} (run `python -m yanchor_amd.build`)")
    return _native.lib()


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"


def test_every_declared_entry_point_has_a_binding():
    bound = set(_native.SIGNATURES) | set(_native.PLAIN) | {"yh_last_error", "yh_abi_version"}
    assert set(declared_symbols()) <= bound


def test_abi_version(lib):
    assert lib.yh_abi_version() == _native.ABI_VERSION


def test_invalid_arguments_return_error_without_device_work(lib):
    # null pointers are rejected before any HIP call
    rc = lib.yh_gdn_recurrent(None, None, None, None, None, None, None, None, 1, 1, 1, 1, 128, 128, 1,
                              1.0, 1, 1, 0, 0, None)
    assert rc == -1
    assert b"null" in lib.yh_last_error()
    # a K the kernels do not support is rejected with a message
    fake = ctypes.c_void_p(16)
    rc = lib.yh_gdn_recurrent(fake, fake, fake, fake, fake, fake, None, fake, 1, 1, 1, 1, 96, 128, 1,
                              1.0, 1, 1, 0, 0, None)
    assert rc == -1 and b"K must be" in lib.yh_last_error()
    rc = lib.yh_gdn_recurrent(fake, fake, fake, fake, fake, fake, None, fake, 1, 1, 3, 4, 128, 128, 1,
                              1.0, 1, 1, 0, 0, None)
    assert rc == -1 and b"multiple" in lib.yh_last_error()


def test_wrappers_reject_host_tensors():
    """The product path never falls back to a host computation."""
    import torch
    from yanchor_amd import gdn, layers, workloads
    x = workloads.gdn_inputs(1, 1, 1, 1, 64, 64)
    with pytest.raises(ValueError, match="ROCm device"):
        gdn.recurrent_gated_delta_rule(x.q, x.k, x.v, g=x.g, beta=x.beta, initial_state=x.state)
    with pytest.raises(ValueError, match="ROCm device"):
        layers.silu_mul(torch.zeros(2, 16, dtype=torch.bfloat16))


def test_hbm_stream_rejects_bad_arguments(lib):
    fake = ctypes.c_void_p(256)
    assert lib.yh_hbm_stream(4, 0, fake, fake, 1024, 8, None) == -1
    assert b"kind" in lib.yh_last_error()
    assert lib.yh_hbm_stream(0, 0, fake, fake, 1000, 8, None) == -1
    assert b"multiple of 16" in lib.yh_last_error()
    assert lib.yh_hbm_stream(0, 0, None, fake, 1024, 8, None) == -1
    assert b"null" in lib.yh_last_error()
    assert lib.yh_hbm_stream(2, 0, fake, fake, 16, 8, None) == -1
    assert b"grid floats" in lib.yh_last_error()


def test_sampler_refuses_top_k_past_the_vocabulary(lib):
    """top_k > V is refused in every branch, the full-vocabulary one (top_k
    > 64) included, as the reference's top_k_top_p_distribution refuses it
    (runtime/model/inference_kernels.py:46-47); the wrapper refuses it
    before the C ABI is reached."""
    import torch
    from yanchor_amd import inference_kernels as ik
    fake = ctypes.c_void_p(256)
    args = lambda k, v: (fake, _native.F32, v, None, 0, 0.0, fake, None, 0, 1, 0, 1.0, k, 1.0,  # noqa: E731
                         ik.SAMPLE_TORCH, fake, None, None, fake, 1 << 20, 1, v, None)
    assert lib.yh_topk_sample(*args(100, 80)) == -1
    assert b"exceeds the vocabulary" in lib.yh_last_error()
    assert lib.yh_topk_sample(*args(30, 20)) == -1
    assert b"exceeds the vocabulary" in lib.yh_last_error()
    scores = torch.zeros(2, 80)
    ids = torch.zeros(2, dtype=torch.int64)
    for k in (100, 81):
        with pytest.raises(ValueError, match="exceeds the vocabulary"):
            ik.topk_sample(scores, ids, 0, seed=1, temperature=1.0, top_k=k, top_p=1.0, mode=ik.SAMPLE_TORCH)


def test_norm_and_reduce_argument_checks(lib):
    """yh_rmsnorm_partials: a second projection's partials replace the
    projection residual and count toward the 64-plane limit; out2 rows hold
    at least D.  yh_linear_reduce: its 16- and 8-byte accesses need aligned
    pointers.  All refused before any device work."""
    fake = ctypes.c_void_p(256)

    def norm(proj_res, part2, s, s2, out2_stride=2560):
        return lib.yh_rmsnorm_partials(fake, s, proj_res, 2560, part2, s2, None, None, fake, fake, 2560, 4, 2560,
                                       1e-6, 1, fake, fake, out2_stride, None)
    assert norm(fake, fake, 12, 12) == -1 and b"part2 replaces proj_residual" in lib.yh_last_error()
    assert norm(None, fake, 40, 25) == -1 and b"S + S2 <= 64" in lib.yh_last_error()
    assert norm(None, fake, 12, 0) == -1 and b"1 <= S2" in lib.yh_last_error()
    assert norm(None, None, 12, 0, out2_stride=2048) == -1 and b"out2_stride >= D" in lib.yh_last_error()
    odd = ctypes.c_void_p(256 + 8)
    assert lib.yh_linear_reduce(odd, fake, 2560, 4, 2560, 12, None, 0, None) == -1
    assert b"aligned" in lib.yh_last_error()
    assert lib.yh_linear_reduce(fake, ctypes.c_void_p(256 + 2), 2560, 4, 2560, 12, None, 0, None) == -1
    assert lib.yh_linear_reduce(fake, fake, 2560, 4, 2560, 12, ctypes.c_void_p(256 + 4), 2560, None) == -1
