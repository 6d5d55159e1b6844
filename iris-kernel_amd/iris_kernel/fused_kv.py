"""Fused RoPE + INT4 paged append on MI355X (gfx950), and the module's other
two write paths.

Drop-in for ``iris_kernel.fused_kv`` of Hunter2030ZeRo/Iris-Kernel:
``fused_rope_int4_paged_append`` keeps the signature, the validation order,
the exception types and the in-place contract of the reference wrapper
(src/iris_kernel/fused_kv.py:600-780).  The TileLang kernel launch
(fused_kv.py:766-780) is replaced by the HIP kernel of
``csrc/append.hip`` through the C ABI ``iris_rope_int4_paged_append``.

Differences, all on the host side:
* the data-dependent checks (duplicate slots, slot range, position range,
  fused_kv.py:741-759) raise the same errors in the same order but cost one
  device-to-host copy instead of four;
* inputs must be dense; read-only inputs that are not are copied, caches
  that are not raise ``ValueError`` (the reference silently assumes density).

``fused_rope_fp16_append`` (fused_kv.py:153-297, RoPE(K) and V into an fp16
cache, partial rotary_dim allowed) and ``fused_quantize_pack_int4``
(fused_kv.py:365-416, group-32 quantise + pack of a dense tensor) keep the
reference signatures, checks and exceptions the same way, over the HIP
kernels of ``csrc/kv_fp16.hip`` (``iris_rope_fp16_paged_append``,
``iris_quantize_pack_int4``).
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["fused_rope_int4_paged_append", "_rope_int4_paged_append", "fused_rope_fp16_append",
           "_rope_fp16_paged_append", "fused_quantize_pack_int4", "_quantize_pack_int4_g32"]


def _dense(t: torch.Tensor, align: int) -> torch.Tensor:
    if t.is_contiguous() and t.data_ptr() % align == 0:
        return t
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    out.copy_(t)
    return out


def _require_dense(name: str, t: torch.Tensor, align: int) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")


def _launch_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_data, v_data,
                   k_scale, v_scale, head_dim: int, rotary_dim: int, page_size: int) -> None:
    if key.shape[0] == 0 or cos_cache.shape[0] == 0:
        return  # nothing to write (an empty RoPE table admits no valid token)
    key = _dense(key, 16)
    value = _dense(value, 16)
    positions = _dense(positions, 4)
    slot_mapping = _dense(slot_mapping, 4)
    cos_cache = _dense(cos_cache, 16)
    sin_cache = _dense(sin_cache, 16)
    _require_dense("k_data", k_data, 16)
    _require_dense("v_data", v_data, 16)
    _require_dense("k_scale", k_scale, 4)
    _require_dense("v_scale", v_scale, 4)
    stream = _lib.raw_stream(key.device)
    status = _lib.lib().iris_rope_int4_paged_append(
        key.data_ptr(), value.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(),
        cos_cache.data_ptr(), sin_cache.data_ptr(), k_data.data_ptr(), v_data.data_ptr(),
        k_scale.data_ptr(), v_scale.data_ptr(), key.shape[0], key.shape[1], head_dim, rotary_dim,
        page_size, k_data.shape[0], cos_cache.shape[0], stream)
    _lib.check(status, "iris_rope_int4_paged_append")


def fused_rope_int4_paged_append(
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    slot_mapping: torch.Tensor,
    cos_cache: torch.Tensor,
    sin_cache: torch.Tensor,
    k_data: torch.Tensor,
    v_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    *,
    rotary_dim: int,
    group_size: int = 32,
    page_size: int,
) -> None:
    """RoPE(K), quantise K and V to group-32 INT4, pack, scatter into the pages.

    Bit-identical to ``torch_eager_append`` for the scope it accepts
    (fp16, head_dim a multiple of 32 up to 512, group_size == 32, any even
    rotary_dim <= head_dim: the first rotary_dim dims of K are rotated, the
    rest pass through, as the eager path does; the reference's fused kernel
    requires head_dim % 64 == 0 and rotary_dim == head_dim).
    Slots < 0 are skipped.  Mutates k_data/v_data/k_scale/v_scale in place;
    the launch is asynchronous on the current stream.
    """
    # Validation order and messages follow fused_kv.py:616-764.
    if not torch.cuda.is_available():
        raise RuntimeError("Iris fused kernels require CUDA")
    if key.device.type != "cuda":
        raise ValueError("key/value must be CUDA tensors")
    if key.shape != value.shape:
        raise ValueError("key and value must have identical shapes")
    if key.ndim != 3:
        raise ValueError("key/value must have shape [T, Hkv, D]")
    if key.dtype != torch.float16:
        raise TypeError("key must use FP16(torch.float16)")
    if value.dtype != torch.float16:
        raise TypeError("value must use FP16(torch.float16)")
    num_tokens, num_kv_heads, head_dim = key.shape
    # head_dim: every multiple of the 32-dim scale group up to 512, as the
    # eager path takes it (the reference's fused path: multiples of 64).
    if head_dim <= 0 or head_dim % 32 != 0 or head_dim > 512:
        raise NotImplementedError("Stage C currently requires head_dim divisible by 32 (at most 512)")
    if group_size != 32:
        raise NotImplementedError("Stage C currently supports group_size=32")
    # Partial RoPE is accepted (the eager path's rule, torch_eager_kv.py:35-49,
    # where the reference's fused path raises NotImplementedError).
    if rotary_dim < 0:
        raise ValueError("rotary_dim must be non-negative")
    if rotary_dim > head_dim:
        raise ValueError("rotary_dim cannot exceed head_dim")
    if rotary_dim % 2 != 0:
        raise ValueError("rotary_dim must be even")
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    if positions.shape != (num_tokens,):
        raise ValueError("positions must have shape [T]")
    if slot_mapping.shape != (num_tokens,):
        raise ValueError("slot_mapping must have shape [T]")
    device = key.device
    for name, tensor in (("value", value), ("positions", positions), ("slot_mapping", slot_mapping),
                         ("cos_cache", cos_cache), ("sin_cache", sin_cache), ("k_data", k_data),
                         ("v_data", v_data), ("k_scale", k_scale), ("v_scale", v_scale)):
        if tensor.device != device:
            raise ValueError(f"{name} must be on {device}")
    if positions.dtype != torch.int32:
        raise TypeError("positions must use torch.int32")
    if slot_mapping.dtype != torch.int32:
        raise TypeError("slot_mapping must use torch.int32")
    half = rotary_dim // 2
    if cos_cache.ndim != 2:
        raise ValueError("cos_cache must have shape [max_position, rotary_dim // 2]")
    if sin_cache.shape != cos_cache.shape:
        raise ValueError("sin_cache must match cos_cache")
    if cos_cache.shape[-1] != half:
        raise ValueError(f"RoPE cache width must be {half}")
    if cos_cache.dtype != torch.float16:
        raise TypeError("cos_cache must use FP16(torch.float16)")
    if sin_cache.dtype != torch.float16:
        raise TypeError("sin_cache must use FP16(torch.float16)")
    if k_data.ndim != 4:
        raise ValueError("k_data/v_data must be rank-4 tensors")
    num_pages = k_data.shape[0]
    data_shape = (num_pages, page_size, num_kv_heads, head_dim // 2)
    scale_shape = (num_pages, page_size, num_kv_heads, head_dim // group_size)
    if tuple(k_data.shape) != data_shape:
        raise ValueError(f"k_data must have shape {data_shape}")
    if tuple(v_data.shape) != data_shape:
        raise ValueError(f"v_data must have shape {data_shape}")
    if tuple(k_scale.shape) != scale_shape:
        raise ValueError(f"k_scale must have shape {scale_shape}")
    if tuple(v_scale.shape) != scale_shape:
        raise ValueError(f"v_scale must have shape {scale_shape}")
    if k_data.dtype != torch.uint8:
        raise TypeError("k_data must use UINT8(torch.uint8)")
    if v_data.dtype != torch.uint8:
        raise TypeError("v_data must use UINT8(torch.uint8)")
    if k_scale.dtype != torch.float16:
        raise TypeError("k_scale must use FP16(torch.float16)")
    if v_scale.dtype != torch.float16:
        raise TypeError("v_scale must use FP16(torch.float16)")

    if head_dim > 512:
        raise NotImplementedError("the gfx950 append kernel supports head_dim <= 512")

    # Data-dependent checks of fused_kv.py:741-759, in the same order: one
    # device launch and one device-to-host copy.
    any_valid, has_dup, slot_oob, pos_neg, pos_oob = _slot_flags(
        slot_mapping, positions, num_pages * page_size, cos_cache.shape[0], device)
    if any_valid:
        if has_dup:
            raise ValueError("duplicate physical KV-cache slots are not allowed")
        if slot_oob:
            raise IndexError("slot_mapping points outside allocated KV cache")
        if pos_neg:
            raise IndexError("positions must be non-negative")
        if pos_oob:
            raise IndexError("positions point outside RoPE cache")

    capability = torch.cuda.get_device_capability(device)
    if capability < (7, 0):
        raise RuntimeError(f"unsupported CUDA compute capability: {capability}")
    if not any_valid:
        return  # the kernel would skip every token
    _launch_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_data, v_data,
                   k_scale, v_scale, head_dim, rotary_dim, page_size)


def _rope_int4_paged_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_data,
                            v_data, k_scale, v_scale, head_dim: int, page_size: int,
                            threads: int = 64) -> None:
    """Positional kernel handle with the reference's call shape
    (fused_kv.py:419-434; called directly by the reference's tests/bench.py).
    No validation and no host synchronisation; ``threads`` is accepted and
    ignored (the HIP launch shape is fixed by the kernel)."""
    del threads
    _launch_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_data, v_data,
                   k_scale, v_scale, head_dim, head_dim, page_size)


# ------------------------------------------------------- FP16 cache append


_CHECK_BUFFERS: dict[tuple[int, int], tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = {}


def _check_buffers(device, num_slots: int, stream: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """iris_append_check's state (16 int64) and slot bitmap for `stream`,
    zero-filled when made (each launch leaves them zero), and the pinned
    host buffer that receives its results."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    words = max(1, (num_slots + 31) // 32)
    bufs = _CHECK_BUFFERS.get(key)
    if bufs is None or bufs[1].numel() < words:
        state = bufs[0] if bufs is not None else torch.zeros(16, dtype=torch.int64, device=device)
        host = bufs[2] if bufs is not None else torch.zeros(8, dtype=torch.int64, pin_memory=True)
        bufs = (state, torch.zeros(words, dtype=torch.int32, device=device), host)
        _CHECK_BUFFERS[key] = bufs
    return bufs


def _slot_flags(slot_mapping, positions, num_slots: int, num_positions: int, device) -> list:
    """[any valid slot, duplicate valid slot, valid slot >= num_slots, valid
    position < 0, valid position >= num_positions] (slots < 0 are skipped
    tokens): one iris_append_check launch and one device-to-host copy.  With
    a slot outside the cache, the duplicate test over every valid slot
    (which the reference reports first) is redone with torch operations."""
    stream = _lib.raw_stream(device)
    state, bitmap, host = _check_buffers(device, num_slots, stream)
    sl = _dense(slot_mapping, 4)
    pos = _dense(positions, 4)
    _lib.check(_lib.lib().iris_append_check(sl.data_ptr(), pos.data_ptr(), sl.numel(), num_slots, num_positions,
                                            state.data_ptr(), bitmap.data_ptr(), bitmap.numel(), host.data_ptr(),
                                            stream),
               "iris_append_check")  # returns once the results are in `host`
    flags = host[:5].tolist()
    if flags[2]:
        return _slot_flags_torch(slot_mapping, positions, num_slots, num_positions, device)
    return flags


def _slot_flags_torch(slot_mapping, positions, num_slots: int, num_positions: int, device) -> list:
    """_slot_flags with torch operations (a sort finds the duplicates)."""
    valid = slot_mapping >= 0
    big = torch.iinfo(torch.int64).max
    vs = torch.where(valid, slot_mapping.to(torch.int64), big)
    sorted_slots, _ = torch.sort(vs)
    dup = ((sorted_slots[1:] == sorted_slots[:-1]) & (sorted_slots[1:] != big)).any() \
        if slot_mapping.numel() > 1 else torch.zeros((), dtype=torch.bool, device=device)
    return torch.stack([
        valid.any(),
        dup,
        (valid & (slot_mapping.to(torch.int64) >= num_slots)).any(),
        (valid & (positions < 0)).any(),
        (valid & (positions >= num_positions)).any(),
    ]).cpu().tolist()


def _launch_fp16_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_cache, v_cache,
                        head_dim: int, rotary_dim: int, page_size: int) -> None:
    if key.shape[0] == 0:
        return
    key = _dense(key, 16)
    value = _dense(value, 16)
    positions = _dense(positions, 4)
    slot_mapping = _dense(slot_mapping, 4)
    cos_cache = _dense(cos_cache, 16)
    sin_cache = _dense(sin_cache, 16)
    _require_dense("k_cache", k_cache, 2)
    _require_dense("v_cache", v_cache, 2)
    stream = _lib.raw_stream(key.device)
    status = _lib.lib().iris_rope_fp16_paged_append(
        key.data_ptr(), value.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(),
        cos_cache.data_ptr(), sin_cache.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        key.shape[0], key.shape[1], head_dim, rotary_dim, page_size, k_cache.shape[0],
        cos_cache.shape[0], stream)
    _lib.check(status, "iris_rope_fp16_paged_append")


def fused_rope_fp16_append(
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    slot_mapping: torch.Tensor,
    cos_cache: torch.Tensor,
    sin_cache: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    *,
    rotary_dim: int,
    page_size: int,
) -> None:
    """RoPE(K) on the first ``rotary_dim`` dims, then K and V into the fp16
    cache [NP, page_size, Hkv, D] at their slots (slots < 0 are skipped).
    The written rows are bit-identical to ``apply_rope``'s.  Mutates
    k_cache/v_cache in place; asynchronous on the current stream."""
    # Validation order and messages follow fused_kv.py:166-282.
    if not torch.cuda.is_available():
        raise RuntimeError("Iris fused kernels require CUDA")
    if key.device.type != "cuda":
        raise ValueError("key/value must be CUDA tensors")
    if key.shape != value.shape:
        raise ValueError("key and value must have identical shapes")
    if key.ndim != 3:
        raise ValueError("key/value must have shape [T, Hkv, D]")
    if key.dtype != torch.float16:
        raise TypeError("Stage A currently supports FP16 input")
    if value.dtype != torch.float16:
        raise TypeError("Stage A currently supports FP16 input")
    num_tokens, num_kv_heads, head_dim = key.shape
    if rotary_dim > head_dim:
        raise ValueError("rotary_dim cannot exceed head_dim")
    if rotary_dim % 2 != 0:
        raise ValueError("rotary_dim must be even")
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    if positions.shape != (num_tokens,):
        raise ValueError("positions must have shape [T]")
    if slot_mapping.shape != (num_tokens,):
        raise ValueError("slot_mapping must have shape [T]")
    if tuple(k_cache.shape[1:]) != (page_size, num_kv_heads, head_dim):
        raise ValueError("invalid k_cache shape")
    if tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError("k_cache and v_cache must have identical shapes")
    if k_cache.dtype != torch.float16:
        raise TypeError("Stage A cache must use FP16")
    if v_cache.dtype != torch.float16:
        raise TypeError("Stage A cache must use FP16")
    device = key.device
    for name, tensor in (("value", value), ("positions", positions), ("slot_mapping", slot_mapping),
                         ("cos_cache", cos_cache), ("sin_cache", sin_cache), ("k_cache", k_cache),
                         ("v_cache", v_cache)):
        if tensor.device != device:
            raise ValueError(f"{name} must be on {device}")
    if positions.dtype != torch.int32:
        raise TypeError("positions must use torch.int32")
    if slot_mapping.dtype != torch.int32:
        raise TypeError("slot_mapping must use torch.int32")
    half = rotary_dim // 2
    if cos_cache.ndim != 2:
        raise ValueError("cos_cache must have shape [max_position, rotary_dim // 2]")
    if sin_cache.shape != cos_cache.shape:
        raise ValueError("sin_cache must match cos_cache")
    if cos_cache.shape[-1] != half:
        raise ValueError(f"RoPE cache width must be {half}")
    if cos_cache.dtype != torch.float16:
        raise TypeError("Stage A RoPE cache must use FP16")
    if sin_cache.dtype != torch.float16:
        raise TypeError("Stage A RoPE cache must use FP16")
    capability = torch.cuda.get_device_capability(device)
    if capability < (7, 0):
        raise RuntimeError(f"unsupported CUDA compute capability: {capability}")
    # Data-dependent checks of fused_kv.py:263-282, same order, one copy.
    any_valid, has_dup, slot_oob, pos_neg, pos_oob = _slot_flags(
        slot_mapping, positions, k_cache.shape[0] * page_size, cos_cache.shape[0], device)
    if any_valid:
        if has_dup:
            raise ValueError("duplicate physical KV-cache slots are not allowed")
        if slot_oob:
            raise IndexError("slot_mapping points outside allocated cache")
    if pos_neg:
        raise IndexError("positions must be non-negative")
    if pos_oob:
        raise IndexError("positions point outside RoPE cache")
    if not any_valid:
        return
    _launch_fp16_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_cache, v_cache,
                        head_dim, rotary_dim, page_size)


def _rope_fp16_paged_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_cache, v_cache,
                            head_dim: int, rotary_dim: int, page_size: int, threads: int = 64) -> None:
    """Positional kernel handle with the reference's call shape
    (fused_kv.py:9-22); no validation, ``threads`` ignored."""
    del threads
    _launch_fp16_append(key, value, positions, slot_mapping, cos_cache, sin_cache, k_cache, v_cache,
                        head_dim, rotary_dim, page_size)


# ----------------------------------------------------- standalone quantiser


def _launch_quantize_pack(x, packed, scales, head_dim: int) -> None:
    if x.numel() == 0:
        return
    x = _dense(x, 16)
    _require_dense("packed", packed, 4)
    _require_dense("scales", scales, 2)
    stream = _lib.raw_stream(x.device)
    status = _lib.lib().iris_quantize_pack_int4(x.data_ptr(), packed.data_ptr(), scales.data_ptr(),
                                                x.shape[0], x.shape[1], head_dim, stream)
    _lib.check(status, "iris_quantize_pack_int4")


def fused_quantize_pack_int4(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> None:
    """Group-32 INT4 quantisation and packing of x [T, H, D] fp16 into
    packed [T, H, D/2] uint8 and scales [T, H, D/32] fp16, bit-identical to
    ``pack_int4(quantize_int4_groupwise(x, 32))``; asynchronous on the
    current stream.  Checks follow fused_kv.py:370-408."""
    if not torch.cuda.is_available():
        raise RuntimeError("Iris fused kernels require CUDA")
    if x.device.type != "cuda":
        raise ValueError("x must be a CUDA tensor")
    if x.ndim != 3:
        raise ValueError("x must have shape [T, H_kv, D]")
    if x.dtype != torch.float16:
        raise TypeError("INT4 fast path currently requires FP16 input")
    _, _, head_dim = x.shape
    if head_dim % 64 != 0:
        raise NotImplementedError("INT4 fast path currently requires head_dim divisible by 64")
    expected_packed = (x.shape[0], x.shape[1], head_dim // 2)
    expected_scales = (x.shape[0], x.shape[1], head_dim // 32)
    if tuple(packed.shape) != expected_packed:
        raise ValueError(f"packed tensor must have shape {expected_packed}")
    if tuple(scales.shape) != expected_scales:
        raise ValueError(f"scales must have shape {expected_scales}")
    if packed.dtype != torch.uint8:
        raise TypeError("packed tensor must use UINT8(torch.uint8)")
    if scales.dtype != torch.float16:
        raise TypeError("scales must use FP16(torch.float16)")
    if packed.device != x.device:
        raise ValueError("packed tensor must be on the same device as x")
    if scales.device != x.device:
        raise ValueError("scales must be on the same device as x")
    if head_dim > 512:
        raise NotImplementedError("the gfx950 quantise-pack kernel supports head_dim <= 512")
    _launch_quantize_pack(x, packed, scales, head_dim)


def _quantize_pack_int4_g32(x, packed, scales, head_dim: int, threads: int = 64) -> None:
    """Positional kernel handle with the reference's call shape
    (fused_kv.py:301-307); no validation, ``threads`` ignored."""
    del threads
    _launch_quantize_pack(x, packed, scales, head_dim)
