"""ctypes binding of libiris_hip.so (declared in include/iris_hip.h).

The library is loaded after ``import torch``, so its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded: tensors, streams
and kernels share one runtime.  There is no fallback: if the library is
missing or fails to load, every fused entry point raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime first)

LIB_PATH = Path(__file__).resolve().with_name("libiris_hip.so")

IRIS_OK = 0
_STATUS = {
    1: "invalid argument (shape or size outside the supported scope)",
    2: "HIP kernel launch failed",
    3: "split-KV workspace missing or too small",
}

_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

_SIGNATURES = {
    "iris_rope_int4_paged_append": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                    _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "iris_decode_plan": [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                         ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i32),
                         ctypes.POINTER(_i64)],
    "iris_int4_paged_decode_attention": [_p, _p, _p, _p, _p, _p, _p, _p, _i32, _p, _i64,
                                         _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                         ctypes.c_float, _i32, _i32, _i32, _p],
    "iris_int4_paged_decode_attention_noalloc": [_p, _p, _p, _p, _p, _p, _p, _p, _i32, _i64,
                                                 _i64, _i64, _i64, _i64, _i64, _i64,
                                                 ctypes.c_float, _i32, _i32, _i32, _p],
    "iris_fp16_decode_plan": [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                              ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i64)],
    "iris_fp16_paged_decode_attention": [_p, _p, _p, _p, _p, _p, _i32, _p, _i64,
                                         _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                         ctypes.c_float, _i32, _i32, _p],
    "iris_rope_fp16_paged_append": [_p, _p, _p, _p, _p, _p, _p, _p,
                                    _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "iris_quantize_pack_int4": [_p, _p, _p, _i64, _i64, _i64, _p],
    "iris_decode_check": [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _p],
    "iris_append_check": [_p, _p, _i64, _i64, _i64, _p, _p, _i64, _p, _p],
    "iris_version": [],
}


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m iris_kernel._build` "
                "(or __graft_entry__.build()) first"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != IRIS_OK:
        raise RuntimeError(f"{what}: {_STATUS.get(status, f'status {status}')}")


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def raw_stream(device) -> int:
    """The current HIP stream of `device` as an integer handle (torch's
    current-stream accessor without building a Stream object)."""
    import torch

    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)
