"""Eager PyTorch write path of the compressed paged KV cache.

The drop-in counterpart of ``iris_kernel.torch_eager_kv`` in
Hunter2030ZeRo/Iris-Kernel (src/iris_kernel/torch_eager_kv.py): the same
four functions, signatures, validation order, exception types and results,
in plain PyTorch on any device.  It is the readable definition of the cache
format that callers (and the reference's own tests and benches) compare the
fused HIP path against; the fused path (``iris_kernel.fused_kv``) never calls
it.

The arithmetic that decides bits is the reference's, op for op:

* RoPE: rotate-half over the first ``rotary_dim`` dims in the input dtype,
  every product and every sum a separately rounded tensor op;
* quantisation: fp32 group amax, IEEE ``amax / 7``, clamped to
  ``finfo(dtype).tiny``, rounded to the input dtype, then the fp32 values
  divided by that stored scale, rounded half to even and clamped to [-7, 7];
* packing: the even dim in the low nibble, two's complement.
"""
from __future__ import annotations

import torch

__all__ = ["apply_rope", "quantize_int4_groupwise", "pack_int4", "torch_eager_append"]


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rotary_dim: int) -> torch.Tensor:
    """Rotate-half RoPE on ``x[..., :rotary_dim]``; the other dims pass through.

    torch_eager_kv.py:6-49: with ``x1, x2`` the two halves of the rotated
    part, ``(x1 cos - x2 sin, x2 cos + x1 sin)``; cos and sin are
    ``[..., rotary_dim // 2]`` and broadcast against ``x``.
    """
    if x.ndim < 1:
        raise ValueError("x must have at least one dimension")
    if rotary_dim < 0:
        raise ValueError("rotary_dim must be non-negative")
    if rotary_dim > x.shape[-1]:
        raise ValueError(f"rotary_dim ({rotary_dim}) cannot exceed head_dim ({x.shape[-1]})")
    if rotary_dim % 2 != 0:
        raise ValueError("rotary_dim must be even")
    if rotary_dim == 0:
        return x
    half = rotary_dim // 2
    if cos.shape[-1] != half or sin.shape[-1] != half:
        raise ValueError(f"cos/sin width must be rotary_dim // 2 ({half})")
    rot, rest = x[..., :rotary_dim], x[..., rotary_dim:]
    x1, x2 = rot.chunk(2, dim=-1)
    # rotate_half(rot) = (-x2, x1); the negation is exact, so
    # rot * (cos, cos) + rotate_half(rot) * (sin, sin) rounds exactly as
    # x1 cos - x2 sin and x2 cos + x1 sin do.
    turned = torch.cat((-x2, x1), dim=-1)
    cos2 = torch.cat((cos, cos), dim=-1)
    sin2 = torch.cat((sin, sin), dim=-1)
    out = rot * cos2 + turned * sin2
    return torch.cat((out, rest), dim=-1) if rest.shape[-1] else out


def quantize_int4_groupwise(x: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-group INT4 codes (int8 in [-7, 7]) and scales (x.dtype).

    torch_eager_kv.py:52-88.
    """
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    if x.shape[-1] % group_size != 0:
        raise ValueError(
            f"last dimension ({x.shape[-1]}) must be divisible by group_size ({group_size})"
        )
    groups = x.float().unflatten(-1, (x.shape[-1] // group_size, group_size))
    amax = groups.abs().amax(dim=-1, keepdim=True)
    scale = torch.clamp_min(amax / 7.0, torch.finfo(x.dtype).tiny).to(x.dtype)
    codes = torch.clamp(torch.round(groups / scale.float()), -7, 7).to(torch.int8)
    return codes.flatten(-2), scale.squeeze(-1)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """int8 codes in [-7, 7] -> uint8, two per byte, even index in the low nibble.

    torch_eager_kv.py:91-107.
    """
    if q.dtype != torch.int8:
        raise TypeError(f"q must have dtype torch.int8, got {q.dtype}")
    if q.shape[-1] % 2 != 0:
        raise ValueError("last dimension must be even for INT4 packing")
    if bool(((q < -7) | (q > 7)).any()):
        raise ValueError("INT4 values must lie in [-7, 7]")
    pairs = q.unflatten(-1, (q.shape[-1] // 2, 2)).to(torch.uint8) & 0x0F
    return pairs[..., 0] | (pairs[..., 1] << 4)


def _check_append_inputs(key, value, positions, slot_mapping, cos_cache, sin_cache, k_data, v_data,
                         k_scale, v_scale, rotary_dim, group_size, page_size):
    """The checks of torch_eager_kv.py:111-258, in the reference's order."""
    if key.shape != value.shape:
        raise ValueError("key and value must have identical shapes")
    if key.ndim != 3:
        raise ValueError("key/value must have shape [T, Hkv, D]")
    if key.dtype != value.dtype:
        raise TypeError("key and value must have identical dtypes")
    if not key.is_floating_point():
        raise TypeError("key and value must use a floating-point dtype")
    num_tokens, num_heads, head_dim = key.shape
    if positions.shape != (num_tokens,):
        raise ValueError(f"positions must have shape ({num_tokens},), got {tuple(positions.shape)}")
    if slot_mapping.shape != (num_tokens,):
        raise ValueError(f"slot_mapping must have shape ({num_tokens},), got {tuple(slot_mapping.shape)}")
    if rotary_dim < 0:
        raise ValueError("rotary_dim must be non-negative")
    if rotary_dim > head_dim:
        raise ValueError("rotary_dim cannot exceed head_dim")
    if rotary_dim % 2 != 0:
        raise ValueError("rotary_dim must be even")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    if head_dim % group_size != 0:
        raise ValueError("head_dim must be divisible by group_size")
    if head_dim % 2 != 0:
        raise ValueError("head_dim must be even for INT4 packing")
    device = key.device
    others = {"value": value, "cos_cache": cos_cache, "sin_cache": sin_cache, "k_data": k_data,
              "v_data": v_data, "k_scale": k_scale, "v_scale": v_scale}
    for name, t in others.items():
        if t.device != device:
            raise ValueError(f"{name} must be on {device}, got {t.device}")
    if cos_cache.shape != sin_cache.shape:
        raise ValueError("cos_cache and sin_cache must have identical shapes")
    if cos_cache.ndim != 2:
        raise ValueError("cos_cache/sin_cache must have shape [max_position, rotary_dim // 2]")
    if cos_cache.shape[-1] != rotary_dim // 2:
        raise ValueError(f"RoPE cache width must be {rotary_dim // 2}, got {cos_cache.shape[-1]}")
    if k_data.ndim != 4:
        raise ValueError("k_data/v_data must be rank-4 tensors")
    num_pages = k_data.shape[0]
    packed_shape = (num_pages, page_size, num_heads, head_dim // 2)
    scale_shape = (num_pages, page_size, num_heads, head_dim // group_size)
    for name, t, want in (("k_data", k_data, packed_shape), ("v_data", v_data, packed_shape),
                          ("k_scale", k_scale, scale_shape), ("v_scale", v_scale, scale_shape)):
        if tuple(t.shape) != want:
            raise ValueError(f"{name} shape mismatch: expected {want}, got {tuple(t.shape)}")
    if k_data.dtype != torch.uint8:
        raise TypeError(f"k_data must use torch.uint8, got {k_data.dtype}")
    if v_data.dtype != torch.uint8:
        raise TypeError(f"v_data must use torch.uint8, got {v_data.dtype}")
    if k_scale.dtype != key.dtype:
        raise TypeError(f"k_scale dtype must match key dtype ({key.dtype}), got {k_scale.dtype}")
    if v_scale.dtype != key.dtype:
        raise TypeError(f"v_scale dtype must match value dtype ({value.dtype}), got {v_scale.dtype}")
    return num_pages


@torch.no_grad()
def torch_eager_append(
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
    group_size: int,
    page_size: int,
) -> None:
    """RoPE(K), INT4-quantise K and V per group, pack, scatter into the pages.

    torch_eager_kv.py:110-337.  Tokens with ``slot_mapping < 0`` are
    skipped; duplicate valid slots raise ValueError; positions outside the
    RoPE table and slots past the cache raise IndexError.  Only the written
    slots of the four cache tensors change.
    """
    num_pages = _check_append_inputs(key, value, positions, slot_mapping, cos_cache, sin_cache,
                                     k_data, v_data, k_scale, v_scale, rotary_dim, group_size,
                                     page_size)
    device = key.device
    slots = slot_mapping.to(device=device, dtype=torch.int64)
    valid = torch.nonzero(slots >= 0).flatten()
    if valid.numel() == 0:
        return
    slots = slots.index_select(0, valid)
    pos = positions.to(device=device, dtype=torch.int64).index_select(0, valid)
    if slots.unique().numel() != slots.numel():
        raise ValueError("duplicate physical KV-cache slots are not allowed")
    if bool((pos < 0).any()):
        raise IndexError("positions must be non-negative")
    if bool((pos >= cos_cache.shape[0]).any()):
        raise IndexError("positions point outside RoPE cache")
    page, offset = slots.div(page_size, rounding_mode="floor"), slots.remainder(page_size)
    if bool((page >= num_pages).any()):
        raise IndexError("slot_mapping points outside allocated KV cache")

    k = key.index_select(0, valid)
    v = value.index_select(0, valid)
    cos = cos_cache.index_select(0, pos).to(key.dtype)[:, None, :]
    sin = sin_cache.index_select(0, pos).to(key.dtype)[:, None, :]
    k = apply_rope(k, cos, sin, rotary_dim=rotary_dim)
    for src, data, scales in ((k, k_data, k_scale), (v, v_data, v_scale)):
        codes, group_scales = quantize_int4_groupwise(src, group_size=group_size)
        data[page, offset] = pack_int4(codes)
        scales[page, offset] = group_scales
