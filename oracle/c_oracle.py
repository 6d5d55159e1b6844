"""ctypes binding of the C restatement (iris_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Wraps torch CPU tensors as raw pointers.  The library is built by
``oracle/Makefile`` into ``oracle/_build/libiris_oracle.so``; ``load()``
builds it when it is missing.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libiris_oracle.so"

_lib = None
_p = ctypes.c_void_p
_i64 = ctypes.c_int64


def build() -> Path:
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.ior_append.argtypes = [_p] * 10 + [_i64] * 8
        lib.ior_append.restype = ctypes.c_int
        lib.ior_decode.argtypes = [_p] * 7 + [_i64] * 8 + [ctypes.c_double, _p]
        lib.ior_decode.restype = ctypes.c_int
        lib.ior_check_scale_mul.argtypes = []
        lib.ior_check_scale_mul.restype = _i64
        lib.ior_check_quant_grid.argtypes = [ctypes.c_int, ctypes.c_int]
        lib.ior_check_quant_grid.restype = _i64
        lib.ior_check_pack_sum.argtypes = [ctypes.c_int32]
        lib.ior_check_pack_sum.restype = _i64
        lib.ior_f32_to_f16_array.argtypes = [_p, _p, _i64]
        lib.ior_f16_to_f32_array.argtypes = [_p, _p, _i64]
        _lib = lib
    return _lib


def _ptr(t: torch.Tensor) -> int:
    assert t.device.type == "cpu" and t.is_contiguous()
    return t.data_ptr()


APPEND_ERRORS = {
    -1: (ValueError, "duplicate physical KV-cache slots are not allowed"),
    -2: (IndexError, "positions must be non-negative"),
    -3: (IndexError, "positions point outside RoPE cache"),
    -4: (IndexError, "slot_mapping points outside allocated KV cache"),
    -5: (ValueError, "invalid static arguments"),
}

DECODE_ERRORS = {
    -1: (ValueError, "all sequence lengths must be positive"),
    -2: (ValueError, "block_table does not contain enough pages"),
    -3: (IndexError, "block_table contains an invalid physical page id"),
    -5: (ValueError, "invalid static arguments"),
}


def append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_data, v_data, k_scale,
           v_scale, *, rotary_dim: int, group_size: int, page_size: int) -> None:
    """C restatement of torch_eager_append for fp16 tensors (in place)."""
    T, H, D = key.shape
    args = [key.contiguous().view(torch.int16), value.contiguous().view(torch.int16),
            positions.to(torch.int64).contiguous(), slot_mapping.to(torch.int64).contiguous(),
            cos_cache.contiguous().view(torch.int16), sin_cache.contiguous().view(torch.int16)]
    for t in (k_data, v_data, k_scale, v_scale):
        assert t.is_contiguous()
    rc = load().ior_append(*[_ptr(a) for a in args], _ptr(k_data), _ptr(v_data),
                           _ptr(k_scale), _ptr(v_scale), T, H, D, page_size, k_data.shape[0],
                           cos_cache.shape[0], rotary_dim, group_size)
    if rc:
        exc, msg = APPEND_ERRORS[rc]
        raise exc(msg)


def decode_f64(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, *,
               page_size: int = 16, group_size: int = 32,
               softmax_scale: float | None = None) -> torch.Tensor:
    """Float64 brute-force decode attention; returns [B, Hq, D] float64."""
    B, Hq, D = query.shape
    NP, P, Hkv, _ = k_data.shape
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    out = torch.empty((B, Hq, D), dtype=torch.float64)
    args = [query.contiguous().view(torch.int16), k_data.contiguous(), v_data.contiguous(),
            k_scale.contiguous().view(torch.int16), v_scale.contiguous().view(torch.int16),
            block_table.to(torch.int64).contiguous(), seq_lens.to(torch.int64).contiguous()]
    rc = load().ior_decode(*[_ptr(a) for a in args], B, Hq, Hkv, D, P, group_size, NP,
                           block_table.shape[1], float(scale), _ptr(out))
    if rc:
        exc, msg = DECODE_ERRORS[rc]
        raise exc(msg)
    return out


def f32_to_f16_bits(x: torch.Tensor) -> torch.Tensor:
    x = x.to(torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.int16)
    load().ior_f32_to_f16_array(_ptr(x), _ptr(out), x.numel())
    return out


def f16_bits_to_f32(h: torch.Tensor) -> torch.Tensor:
    h = h.to(torch.int16).contiguous()
    out = torch.empty(h.shape, dtype=torch.float32)
    load().ior_f16_to_f32_array(_ptr(h), _ptr(out), h.numel())
    return out


def check_scale_mul() -> int:
    return int(load().ior_check_scale_mul())


def check_quant_grid(rvariant: int, mode: int = 0) -> int:
    """Mismatches of the kernels' two-rounding quantiser (ior_check_quant_grid)."""
    return int(load().ior_check_quant_grid(int(rvariant), int(mode)))


def check_pack_sum(bias_delta: int = 0) -> int:
    """Mismatches of the kernels' shift-and-add nibble packing (ior_check_pack_sum)."""
    return int(load().ior_check_pack_sum(int(bias_delta)))
