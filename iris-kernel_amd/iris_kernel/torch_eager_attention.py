"""Eager PyTorch read path of the compressed paged KV cache.

The drop-in counterpart of ``iris_kernel.torch_eager_attention`` in
Hunter2030ZeRo/Iris-Kernel (src/iris_kernel/torch_eager_attention.py): INT4
unpacking and dequantisation, and GQA decode attention over the paged INT4
cache and over an FP16 paged cache, with the reference's signatures,
validation order and exception types, in plain PyTorch on any device.  The
fused HIP decode (``iris_kernel.fused_attention``) never calls it.

Attention is evaluated for the whole batch at once: the pages of every
sequence are gathered into a ``[B, max_len]`` token axis, tokens past a
sequence's length are masked out of the fp32 softmax, and the result is
rounded to the query dtype -- the reference's per-sequence
``softmax(q . K * scale) . V`` in fp32, batched.
"""
from __future__ import annotations

import torch

__all__ = [
    "unpack_int4",
    "dequantize_int4_groupwise",
    "torch_eager_int4_paged_decode_attention",
    "torch_eager_fp16_paged_decode_attention",
]


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """uint8 ``[..., D/2]`` -> int8 ``[..., D]``, low nibble first, two's complement.

    torch_eager_attention.py:8-26 (a nibble n >= 8 decodes to n - 16).
    """
    if packed.dtype != torch.uint8:
        raise TypeError(f"packed must use torch.uint8, got {packed.dtype}")
    as_signed = packed.view(torch.int8)
    low = torch.bitwise_left_shift(as_signed, 4) >> 4  # arithmetic shift: sign of bit 3
    high = as_signed >> 4
    return torch.stack((low, high), dim=-1).flatten(-2)


def dequantize_int4_groupwise(
    packed: torch.Tensor,
    scales: torch.Tensor,
    *,
    group_size: int = 32,
    dtype: torch.dtype = torch.float16,
) -> torch.Tensor:
    """fp32 code times fp32 group scale, in ``dtype``.  torch_eager_attention.py:29-53."""
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    codes = unpack_int4(packed)
    head_dim = codes.shape[-1]
    if head_dim % group_size != 0:
        raise ValueError("head_dim must be divisible by group_size")
    want = (*codes.shape[:-1], head_dim // group_size)
    if tuple(scales.shape) != want:
        raise ValueError(f"scales must have shape {want}, got {tuple(scales.shape)}")
    grouped = codes.float().unflatten(-1, (head_dim // group_size, group_size))
    return (grouped * scales.float()[..., None]).flatten(-2).to(dtype)


def _validate_attention_inputs(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, *,
                               page_size, group_size):
    """The checks of torch_eager_attention.py:56-151, in the reference's order."""
    if query.ndim != 3:
        raise ValueError("query must have shape [B, Hq, D]")
    if query.dtype != torch.float16:
        raise TypeError("query must use torch.float16")
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    batch, num_q_heads, head_dim = query.shape
    if k_data.ndim != 4:
        raise ValueError("k_data/v_data must have shape [NP, P, Hkv, D/2]")
    if tuple(v_data.shape) != tuple(k_data.shape):
        raise ValueError("k_data and v_data must have identical shapes")
    if k_data.dtype != torch.uint8 or v_data.dtype != torch.uint8:
        raise TypeError("k_data/v_data must use torch.uint8")
    num_pages, cache_page, num_kv_heads, packed_dim = k_data.shape
    if cache_page != page_size:
        raise ValueError("cache page dimension does not match page_size")
    if packed_dim * 2 != head_dim:
        raise ValueError("packed cache head dimension does not match query")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    if head_dim % group_size != 0:
        raise ValueError("head_dim must be divisible by group_size")
    scale_shape = (num_pages, page_size, num_kv_heads, head_dim // group_size)
    if tuple(k_scale.shape) != scale_shape:
        raise ValueError(f"k_scale must have shape {scale_shape}, got {tuple(k_scale.shape)}")
    if tuple(v_scale.shape) != scale_shape:
        raise ValueError(f"v_scale must have shape {scale_shape}, got {tuple(v_scale.shape)}")
    if k_scale.dtype != torch.float16 or v_scale.dtype != torch.float16:
        raise TypeError("k_scale/v_scale must use torch.float16")
    if block_table.ndim != 2 or block_table.shape[0] != batch:
        raise ValueError("block_table must have shape [B, max_pages_per_sequence]")
    if seq_lens.shape != (batch,):
        raise ValueError("seq_lens must have shape [B]")
    tensors = {"k_data": k_data, "v_data": v_data, "k_scale": k_scale, "v_scale": v_scale,
               "block_table": block_table, "seq_lens": seq_lens}
    for name, t in tensors.items():
        if t.device != query.device:
            raise ValueError(f"{name} must be on {query.device}")
    if block_table.dtype not in (torch.int32, torch.int64):
        raise TypeError("block_table must use int32 or int64")
    if seq_lens.dtype not in (torch.int32, torch.int64):
        raise TypeError("seq_lens must use int32 or int64")
    if bool((seq_lens <= 0).any()):
        raise ValueError("all sequence lengths must be positive")
    pages_needed = (seq_lens.to(torch.int64) + page_size - 1).div(page_size, rounding_mode="floor")
    if bool((pages_needed > block_table.shape[1]).any()):
        raise ValueError("block_table does not contain enough pages")
    used = torch.arange(block_table.shape[1], device=block_table.device)[None, :] < pages_needed[:, None]
    ids = block_table.to(torch.int64)
    if bool((used & ((ids < 0) | (ids >= num_pages))).any()):
        raise IndexError("block_table contains an invalid physical page id")
    return batch, num_q_heads, num_kv_heads, head_dim


def _gather_tokens(pool: torch.Tensor, block_table: torch.Tensor, n_pages: int) -> torch.Tensor:
    """``pool[NP, P, ...]`` -> ``[B, n_pages * P, ...]`` through the first n_pages columns
    of the block table (unused columns are clamped to page 0 and masked later)."""
    ids = block_table[:, :n_pages].to(torch.int64).clamp(0, pool.shape[0] - 1)
    tokens = pool.index_select(0, ids.flatten())
    return tokens.reshape(ids.shape[0], n_pages * pool.shape[1], *pool.shape[2:])


def _masked_gqa_decode(query, k, v, seq_lens, scale):
    """fp32 ``softmax(q . K^T * scale) . V`` per (sequence, query head) over the
    first seq_lens[b] tokens.  k, v: ``[B, L, Hkv, D]`` fp32; returns ``[B, Hq, D]`` fp32."""
    batch, num_q_heads, head_dim = query.shape
    num_kv_heads = k.shape[2]
    group = num_q_heads // num_kv_heads
    q = query.float().reshape(batch, num_kv_heads, group, head_dim)
    kt = k.permute(0, 2, 3, 1).contiguous()  # [B, Hkv, D, L]
    vv = v.permute(0, 2, 1, 3).contiguous()  # [B, Hkv, L, D]
    logits = torch.matmul(q, kt) * scale  # [B, Hkv, g, L]
    tokens = torch.arange(k.shape[1], device=k.device)
    beyond = tokens[None, :] >= seq_lens.to(device=k.device, dtype=torch.int64)[:, None]
    logits = logits.masked_fill(beyond[:, None, None, :], float("-inf"))
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    probs = probs.masked_fill(beyond[:, None, None, :], 0.0)  # a masked token never contributes, even if V is NaN
    vv = vv.masked_fill(beyond[:, None, :, None], 0.0)
    return torch.matmul(probs, vv).reshape(batch, num_q_heads, head_dim)


@torch.no_grad()
def torch_eager_int4_paged_decode_attention(
    query: torch.Tensor,
    k_data: torch.Tensor,
    v_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    page_size: int = 16,
    group_size: int = 32,
    softmax_scale: float | None = None,
) -> torch.Tensor:
    """GQA decode attention over the paged INT4 cache (torch_eager_attention.py:154-239).

    Query head h reads kv head ``h // (Hq // Hkv)``; K and V are dequantised
    in fp32; the output has the query's dtype.
    """
    batch, _, _, head_dim = _validate_attention_inputs(
        query, k_data, v_data, k_scale, v_scale, block_table, seq_lens,
        page_size=page_size, group_size=group_size)
    scale = float(head_dim ** -0.5 if softmax_scale is None else softmax_scale)
    out = torch.empty_like(query)
    if batch == 0:  # the reference's per-sequence loop runs zero times
        return out
    # sequences in slices of bounded fp32 K/V size
    longest = int(seq_lens.max())
    per_seq = longest * k_data.shape[2] * head_dim * 8
    step = max(1, min(batch, (1 << 30) // max(per_seq, 1)))
    for b0 in range(0, batch, step):
        b1 = min(batch, b0 + step)
        lens = seq_lens[b0:b1]
        n_pages = -(-int(lens.max()) // page_size)
        bt = block_table[b0:b1]
        k = dequantize_int4_groupwise(_gather_tokens(k_data, bt, n_pages), _gather_tokens(k_scale, bt, n_pages),
                                      group_size=group_size, dtype=torch.float32)
        v = dequantize_int4_groupwise(_gather_tokens(v_data, bt, n_pages), _gather_tokens(v_scale, bt, n_pages),
                                      group_size=group_size, dtype=torch.float32)
        out[b0:b1] = _masked_gqa_decode(query[b0:b1], k, v, lens, scale).to(query.dtype)
    return out


@torch.no_grad()
def torch_eager_fp16_paged_decode_attention(
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    page_size: int = 16,
    softmax_scale: float | None = None,
) -> torch.Tensor:
    """GQA decode attention over an FP16 paged cache ``[NP, P, Hkv, D]``
    (torch_eager_attention.py:242-294), the comparator for INT4 quality."""
    if query.ndim != 3:
        raise ValueError("query must have shape [B, Hq, D]")
    if k_cache.ndim != 4 or tuple(k_cache.shape) != tuple(v_cache.shape):
        raise ValueError("k_cache/v_cache must have identical rank-4 shapes")
    batch, num_q_heads, head_dim = query.shape
    num_pages, cache_page, num_kv_heads, cache_dim = k_cache.shape
    if cache_page != page_size or cache_dim != head_dim:
        raise ValueError("FP16 cache shape does not match query/page_size")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    if block_table.shape[0] != batch or seq_lens.shape != (batch,):
        raise ValueError("invalid block_table or seq_lens shape")
    pages_needed = (seq_lens.to(torch.int64) + page_size - 1).div(page_size, rounding_mode="floor")
    used = torch.arange(block_table.shape[1], device=block_table.device)[None, :] < pages_needed[:, None]
    ids = block_table.to(torch.int64)
    if bool((used & ((ids < 0) | (ids >= num_pages))).any()):
        raise IndexError("block_table contains an invalid page id")
    scale = float(head_dim ** -0.5 if softmax_scale is None else softmax_scale)
    if batch == 0:  # the reference's per-sequence loop runs zero times
        return torch.empty_like(query)
    n_pages = -(-int(seq_lens.max()) // page_size)
    k = _gather_tokens(k_cache, block_table, n_pages).float()
    v = _gather_tokens(v_cache, block_table, n_pages).float()
    return _masked_gqa_decode(query, k, v, seq_lens, scale).to(query.dtype)
