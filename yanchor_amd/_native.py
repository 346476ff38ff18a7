"""ctypes binding of ``lib/libyanchor_amd.so`` (the C ABI in include/yanchor_amd.h).

The library is loaded after torch so that it binds to the HIP runtime torch has
already loaded.  There is no fallback: if the library is missing every kernel
call raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libyanchor_amd.so"
# yh_abi_version() of the library these signatures describe (103: yh_rmsnorm_partials takes
# out2_stride; 104: yh_linear_pack lays K blocks outermost; 105: yh_rmsnorm_partials takes part2;
# 106: yh_gdn_decode_fused takes the state dtype)
ABI_VERSION = 106

F32, BF16, F16, I32, I64, U8 = 0, 1, 2, 3, 4, 5
DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16,
              torch.int32: I32, torch.int64: I64, torch.uint8: U8, torch.bool: U8}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes; every entry point returns int status.
SIGNATURES: dict[str, list] = {
    "yh_gdn_recurrent": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                         _f32, _i32, _i32, _i32, _i32, _p],
    "yh_gdn_recurrent_varlen": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                                _i32, _i32, _i32, _i32, _p],
    "yh_gdn_chunk_varlen": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                            _i32, _i32, _i32, _i32, _p, _i64, _p],
    "yh_proj": [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i32, _i32, _i64, _p, _i64, _p, _p],
    "yh_linear_reduce": [_p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "yh_proj_pick": [_i64, _i64, _i64, _i32, _p, _p],
    "yh_conv_prefill": [_p, _i64, _p, _p, _p, _i64, _i64, _i64, _p, _i32, _p],
    "yh_swa_prefill": [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _p, _i64, _i64,
                       _i64, _i64, _i64, _i64, _i32, _p],
    "yh_ring_fill": [_p, _i64, _p, _i64, _p, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "yh_anchor_read": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "yh_window_attend": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "yh_anchor_commit": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                         _i64, _i64, _i64, _p, _i64, _i64, _i32, _p],
    "yh_anchor_prefix": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "yh_anchor_sequence_commit": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _i32, _p],
    "yh_indexed_gqa": [_p, _p, _p, _p, _i32, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "yh_anchor_sequence_read": [_p, _p, _p, _p, _i32, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                _i32, _p],
    "yh_linear": [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "yh_linear_pack": [_p, _p, _i64, _i64, _i32, _p],
    "yh_linear_packed": [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i32, _i64, _p, _i64, _i32, _p, _p],
    "yh_decode_inputs": [_p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                         _f32, _p],
    "yh_gdn_decode_fused": [_p, _i64, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64, _i64, _i64, _i64, _f32, _i32, _f32, _p],
    "yh_rmsnorm_partials": [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _i32, _p, _p, _i64,
                            _p],
    "yh_ring_write": [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                      _f32, _p],
    "yh_memory_prologue": [_p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                           _i64, _f32, _i64, _i64, _p, _i64, _p],
    "yh_anchor_read_gated": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p,
                             _i32, _p],
    "yh_window_attend_gated": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i32, _p],
    "yh_topk_sample": [_p, _i32, _i64, _p, _i64, _f32, _p, _p, _i64, ctypes.c_uint64, ctypes.c_uint64, _f32,
                       _i64, _f32, _i32, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "yh_topk_sample_noalloc": [_p, _i32, _i64, _p, _i64, _f32, _p, _p, _i64, ctypes.c_uint64, ctypes.c_uint64,
                               _f32, _i64, _f32, _i32, _p, _p, _p, _i64, _i64, _p],
    "yh_presence_penalty": [_p, _p, _i64, _f32, _p],
    "yh_counter_uniform": [_p, _p, _i64, ctypes.c_uint64, ctypes.c_uint64, _p, _i64, _p],
    "yh_decode_bookkeeping": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                              _i64, _i64, _p, _i64, _p],
    "yh_cu_seqlens": [_p, _i32, _p, _i64, _p],
    "yh_select_slots": [_p, _p, _i32, _p, _p, _i64, _p],
    "yh_gather_rows": [_i32, _p, _p, _p, _p, _p, _p, _p, _i64, _p],
    "yh_rmsnorm": [_p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _i32, _p],
    "yh_gdn_decode_prep": [_p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                           _p],
    "yh_gated_rmsnorm": [_p, _p, _i64, _p, _p, _i64, _i64, _i64, _f32, _p],
    "yh_silu_mul": [_p, _i64, _p, _i64, _i64, _p],
    "yh_head_norm_rope": [_p, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _f32, _p],
    "yh_hbm_stream": [_i32, _i32, _p, _p, _i64, _i32, _p],
}

# entry points that do not return a status
PLAIN: dict[str, tuple] = {
    "yh_topk_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "yh_linear_split": (_i32, [_i64, _i64, _i64]),
    "yh_linear_packed_split": (_i32, [_i64, _i64, _i64]),
    "yh_gdn_chunk_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "yh_linear_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "yh_topk_segments": (None, [_i64, _i64, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "yh_proj_config_count": (_i32, []),
    "yh_proj_phase_k": (_i32, [_i32]),
    "yh_proj_columns": (_i32, [_i32]),
}

_lib = None


class NativeError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the native library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"yanchor_amd native library not found at {LIB_PATH}; build it with "
                "`python -m yanchor_amd.build` (hipcc, gfx950)")
        handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        handle.yh_last_error.restype = ctypes.c_char_p
        handle.yh_last_error.argtypes = []
        handle.yh_abi_version.restype = ctypes.c_int
        found = handle.yh_abi_version()
        if found != ABI_VERSION:
            raise RuntimeError(f"yanchor_amd native library at {LIB_PATH} has ABI version {found}, these bindings "
                               f"expect {ABI_VERSION}; rebuild it with `python -m yanchor_amd.build`")
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = ctypes.c_int
            fn.argtypes = args
        for name, (res, args) in PLAIN.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Invoke entry point ``name``; raise NativeError with the library's message on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().yh_last_error().decode(errors="replace")
        raise NativeError(f"{name} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All non-None tensors must live on one ROCm device."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("yanchor_amd kernels take ROCm device tensors "
                             f"(got a tensor on {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev
