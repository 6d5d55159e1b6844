"""INT4 (and matched FP16) paged decode attention on MI355X (gfx950).

Drop-in for ``iris_kernel.fused_attention`` of Hunter2030ZeRo/Iris-Kernel:
``fused_int4_paged_decode_attention`` keeps the signature, validation order,
exception types and output contract of the reference wrapper
(src/iris_kernel/fused_attention.py:437-525, validation :373-434).  The
TileLang launch (fused_attention.py:508-524) is replaced by the HIP kernel
of ``csrc/decode.hip`` (attention with the split-KV combine fused into the
same launch) through the C ABI ``iris_int4_paged_decode_attention``.

Additions, all keyword-only and defaulted so existing calls are unchanged:
``tokens_per_split`` / ``waves_per_block`` override the split heuristic,
``workspace`` supplies the split-KV buffer (its head holds 128 arrival
counters per sequence, which every call leaves at zero; the wrapper zeroes
that region the first time it sees a workspace tensor and whenever a call's
batch exceeds the previous call's with it; nothing else may write it between
calls).  Without one, a
zero-filled workspace is cached per (device, stream), so calls on one stream
share it safely and calls on different streams never do.  An fp32 ``output``
tensor receives the values before the final fp16 rounding (test aid).

``fused_fp16_paged_decode_attention`` is the reference's matched FP16
baseline (fused_attention.py:528-582, kernel :223-370) over an fp16 cache
[NP, 16, Hkv, D], backed by ``csrc/decode_fp16.hip`` through
``iris_fp16_paged_decode_attention``; it takes the same additions.
"""
from __future__ import annotations

import ctypes
import weakref

import torch

from . import _lib

__all__ = ["fused_int4_paged_decode_attention", "_int4_paged_decode_attention", "decode_plan",
           "fused_fp16_paged_decode_attention", "_fp16_paged_decode_attention", "fp16_decode_plan",
           "DECODE_PAGE_KERNEL", "DECODE_VALU_TILE", "DECODE_ANY_KERNEL", "DECODE_TOKEN_PAGES",
           "int4_decode_plan"]

# Kernel selection bits or-ed into ``waves_per_block`` (IRIS_DECODE_PAGE_KERNEL
# and IRIS_DECODE_VALU_TILE of include/iris_hip.h), for A/B measurements and
# tests: 16-wave plans keep the general page-streaming kernel, or the general
# kernel runs its VALU tile.  The plan returns them in its wave count, so its
# launch runs the kernel it planned.
DECODE_PAGE_KERNEL = 0x100
DECODE_VALU_TILE = 0x200
# The any-shape kernel (IRIS_DECODE_ANY_KERNEL): every head_dim that is a
# multiple of 32 up to 512, every page size.  The plan picks it by itself for
# head dims other than 64, 96, 128, 160, 192, 224 and 256 (96-224 have an
# MFMA kernel of their own); page sizes that are not a multiple of 16 up to
# 256 ask for DECODE_TOKEN_PAGES (or for it).
DECODE_ANY_KERNEL = 0x400
# The token-page mode of the head-dim MFMA kernel (IRIS_DECODE_TOKEN_PAGES):
# every page size, each token's page looked up through the block table, at
# head_dim 64 to 256 (steps of 32); asked for at other head dims, the plan
# returns the any-shape kernel's.
DECODE_TOKEN_PAGES = 0x800


def decode_plan(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_pages: int,
                total_tokens: int = -1, max_tokens: int = -1, tokens_per_split: int = 0,
                waves_per_block: int = 0) -> tuple[int, int, int, int]:
    """(chunk_tiles, max_chunks, waves_per_block, workspace_bytes) from iris_decode_plan.

    ``max_pages`` counts 16-token pages: ceil(block_table columns * page_size / 16).
    For page sizes that are not a multiple of 16 up to 256 use
    ``int4_decode_plan``, which asks for the token-page mode."""
    ct, mc, nw = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    ws = ctypes.c_int64()
    status = _lib.lib().iris_decode_plan(batch, num_q_heads, num_kv_heads, head_dim, max_pages,
                                         total_tokens, max_tokens, tokens_per_split,
                                         waves_per_block, ctypes.byref(ct), ctypes.byref(mc),
                                         ctypes.byref(nw), ctypes.byref(ws))
    _lib.check(status, "iris_decode_plan")
    return ct.value, mc.value, nw.value, ws.value


def _fast_page_size(page_size: int) -> bool:
    """Page sizes the streaming, MQA, page and general kernels read: 16 m
    for m = 1..16 (a page is m consecutive 16-token pages)."""
    return page_size % 16 == 0 and 16 <= page_size <= 256


def int4_decode_plan(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                     bt_cols: int, total_tokens: int = -1, max_tokens: int = -1, tokens_per_split: int = 0,
                     waves_per_block: int = 0) -> tuple[int, int, int, int]:
    """The decode plan for a cache of ``page_size``-token pages and a block
    table ``bt_cols`` columns wide: ``decode_plan`` over the tokens a row
    addresses.  A page size that is not a multiple of 16 up to 256 asks for
    the token-page mode (which falls back to the any-shape kernel at shapes
    it does not take), or keeps DECODE_ANY_KERNEL if the caller asked for
    that."""
    if not _fast_page_size(page_size):
        sel = DECODE_ANY_KERNEL if waves_per_block > 0 and waves_per_block & DECODE_ANY_KERNEL else DECODE_TOKEN_PAGES
        waves_per_block = (max(waves_per_block, 0) & 0xFF) | sel
    return decode_plan(batch, num_q_heads, num_kv_heads, head_dim, -(-bt_cols * page_size // 16), total_tokens,
                       max_tokens, tokens_per_split, waves_per_block)


def _qk_scale(head_dim: int, softmax_scale) -> float:
    """The logit scale: the reference wrapper passes 0.0 for None
    (fused_attention.py:523) and its kernel maps 0.0 to head_dim ** -0.5
    (fused_attention.py:50), so None and an explicit 0.0 both mean that."""
    if softmax_scale is None or float(softmax_scale) == 0.0:
        return head_dim ** -0.5
    return float(softmax_scale)


_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _stream_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-filled split-KV workspace of the current stream (grown on demand).

    The kernel's arrival counters live at its start and are back at zero
    when a call completes, so consecutive calls on one stream reuse it."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), _lib.raw_stream(device))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


_CHECK_STATES: dict[tuple[int, int], tuple[torch.Tensor, torch.Tensor]] = {}


def _check_state(device: torch.device, stream: int) -> tuple[torch.Tensor, torch.Tensor]:
    """iris_decode_check's state (16 int64 on the device, zero-filled once;
    each launch leaves its accumulators at zero) and the pinned host buffer
    that receives its results, for `stream`."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    bufs = _CHECK_STATES.get(key)
    if bufs is None:
        bufs = (torch.zeros(16, dtype=torch.int64, device=device),
                torch.zeros(8, dtype=torch.int64, pin_memory=True))
        _CHECK_STATES[key] = bufs
    return bufs


_COUNTERS_PER_SEQ = 128  # kCountersPerSeq of csrc/common.h


def counter_region_bytes(batch: int) -> int:
    """Bytes at the head of a split-KV workspace that hold the arrival
    counters of `batch` sequences (the same for every decode kernel)."""
    return (batch * _COUNTERS_PER_SEQ * 4 + 255) // 256 * 256


# id(workspace tensor) -> (data_ptr, bytes, batch): the batch whose counter
# region is known to be zero in that tensor.  An entry lives exactly as long
# as its tensor (a finalizer removes it), so a new tensor that the caching
# allocator places where an old workspace was is never taken for zeroed.
_ZEROED: dict[int, tuple[int, int, int]] = {}


def _ready_workspace(device: torch.device, ws_bytes: int, batch: int,
                     workspace: torch.Tensor | None) -> torch.Tensor:
    """The split-KV workspace for a call, its arrival counters at zero.

    Every kernel keeps its counters at the head of the workspace, 128 per
    sequence, and leaves them at zero; the bytes after them hold partial
    results that each call rewrites.  The first call that sees a workspace
    tensor zero-fills its counter region (one small fill kernel on the
    current stream); later calls with the same tensor object find the
    counters of sequences below the last call's batch at zero and fill only
    when the batch grows.  Between calls the workspace's bytes belong to the
    library: nothing else may write them."""
    if workspace is None:
        workspace = _stream_workspace(device, ws_bytes)
    elif workspace.numel() * workspace.element_size() < ws_bytes:
        raise ValueError(f"workspace must hold at least {ws_bytes} bytes")
    elif not workspace.is_contiguous():
        raise ValueError("workspace must be contiguous")
    key = id(workspace)
    where = (workspace.data_ptr(), workspace.numel() * workspace.element_size())
    entry = _ZEROED.get(key)
    if entry is None or entry[:2] != where or entry[2] < batch:
        workspace.reshape(-1).view(torch.uint8)[:counter_region_bytes(batch)].zero_()
        if entry is None:
            weakref.finalize(workspace, _ZEROED.pop, key, None)
    _ZEROED[key] = (*where, batch)  # the partials of this call may overwrite counters of later sequences
    return workspace


def _launch_decode(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output,
                   softmax_scale: float, plan, workspace=None) -> None:
    chunk_tiles, max_chunks, nw, ws_bytes = plan
    batch, num_q_heads, head_dim = query.shape
    num_pages, page_size, num_kv_heads, _ = k_data.shape
    if ws_bytes > 0:
        workspace = _ready_workspace(query.device, ws_bytes, batch, workspace)
        ws_ptr, ws_len = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    else:
        ws_ptr, ws_len = 0, 0
    for name, t, align in (("query", query, 16), ("k_data", k_data, 16), ("v_data", v_data, 16),
                           ("k_scale", k_scale, 4), ("v_scale", v_scale, 4),
                           ("block_table", block_table, 4), ("seq_lens", seq_lens, 4),
                           ("output", output, 4)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if t.data_ptr() % align:
            raise ValueError(f"{name} must be {align}-byte aligned")
    stream = _lib.raw_stream(query.device)
    status = _lib.lib().iris_int4_paged_decode_attention(
        query.data_ptr(), k_data.data_ptr(), v_data.data_ptr(), k_scale.data_ptr(),
        v_scale.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(), output.data_ptr(),
        1 if output.dtype == torch.float32 else 0, ws_ptr, ws_len, batch, num_q_heads,
        num_kv_heads, head_dim, page_size, num_pages, block_table.shape[1], float(softmax_scale),
        chunk_tiles, max_chunks, nw, stream)
    _lib.check(status, "iris_int4_paged_decode_attention")


# Scope of the INT4 decode beyond the reference's fused path (page_size 16,
# head_dim 64/128, at most 16 query heads per kv head: fused_attention.py:
# 390-403): what its eager path takes (torch_eager_attention.py:72, :93) --
# any page size, any head_dim that is a multiple of the 32-dim scale group
# (up to 512), any GQA ratio.
INT4_MAX_HEAD_DIM = 512


def _validate_common_decode_inputs(query, block_table, seq_lens, *, num_pages: int,
                                   num_kv_heads: int, page_size: int, int4: bool = False):
    """Checks of fused_attention.py:373-434, same order and types; the
    per-sequence page-id loop is one vectorised check.  Returns
    (batch, num_q_heads, head_dim, total_tokens, max_tokens)."""
    if not torch.cuda.is_available():
        raise RuntimeError("Iris fused kernels require CUDA")
    if query.device.type != "cuda":
        raise ValueError("query must be a CUDA tensor")
    if query.ndim != 3:
        raise ValueError("query must have shape [B, Hq, D]")
    if query.dtype != torch.float16:
        raise TypeError("query must use FP16(torch.float16)")
    if (page_size < 1) if int4 else (page_size != 16):
        raise NotImplementedError("decode fast path currently supports page_size="
                                  + ("any positive size" if int4 else "16"))
    batch, num_query_heads, head_dim = query.shape
    if (head_dim % 32 or not 32 <= head_dim <= INT4_MAX_HEAD_DIM) if int4 else head_dim not in (64, 128):
        raise NotImplementedError("decode fast path currently supports head_dim in "
                                  + ("multiples of 32 up to 512" if int4 else "{64, 128}"))
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    if not int4 and num_query_heads // num_kv_heads > 16:
        raise NotImplementedError("decode fast path supports at most 16 query heads per KV head")
    if block_table.ndim != 2 or block_table.shape[0] != batch:
        raise ValueError("block_table must have shape [B, max_pages_per_sequence]")
    if seq_lens.shape != (batch,):
        raise ValueError("seq_lens must have shape [B]")
    # int64 metadata is accepted, as the eager path accepts it
    # (torch_eager_attention.py:130-133; the reference's fused path takes
    # int32 only, fused_attention.py:409-410).
    if block_table.dtype not in (torch.int32, torch.int64) or seq_lens.dtype not in (torch.int32, torch.int64):
        raise TypeError("block_table and seq_lens must use torch.int32 or torch.int64")
    device = query.device
    if block_table.device != device or seq_lens.device != device:
        raise ValueError("block_table and seq_lens must be on the query device")
    if block_table.dtype == torch.int64:
        # ids outside the pool stay outside it (-1 or num_pages), so the
        # device check below reports them as the reference does
        block_table = block_table.clamp(-1, num_pages).to(torch.int32)
    if seq_lens.dtype == torch.int64:
        seq_lens = seq_lens.clamp(-1, 2 ** 31 - 1).to(torch.int32)
    max_pages = block_table.shape[1]
    # The per-sequence checks of fused_attention.py:415-429 (lengths
    # positive, enough pages, page ids inside the pool) in one device
    # launch (iris_decode_check), plus the sum and maximum of the lengths,
    # read back with one copy.
    stream = _lib.raw_stream(device)
    state, host = _check_state(device, stream)
    bt = block_table if block_table.is_contiguous() else block_table.contiguous()
    sl = seq_lens if seq_lens.is_contiguous() else seq_lens.contiguous()
    _lib.check(_lib.lib().iris_decode_check(sl.data_ptr(), bt.data_ptr(), batch, max_pages, num_pages, page_size,
                                            state.data_ptr(), host.data_ptr(), stream),
               "iris_decode_check")  # returns once the results are in `host`
    nonpos, too_few, bad, total, longest = host[:5].tolist()
    if nonpos:
        raise ValueError("all sequence lengths must be positive")
    if too_few:
        raise ValueError("block_table does not contain enough pages")
    if bad:
        raise IndexError("block_table contains an invalid physical page id")
    capability = torch.cuda.get_device_capability(device)
    if capability < (7, 0):
        raise RuntimeError(f"unsupported CUDA compute capability: {capability}")
    return batch, num_query_heads, head_dim, total, longest, bt, sl


def _dense(t: torch.Tensor, align: int) -> torch.Tensor:
    """t itself when contiguous and `align`-byte aligned, else a dense copy
    (a block_table[:, :n] slice or a q split out of a fused qkv projection)."""
    if t.is_contiguous() and t.data_ptr() % align == 0:
        return t
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)  # fresh allocations are 256-byte aligned
    out.copy_(t)
    return out


def fused_int4_paged_decode_attention(
    query: torch.Tensor,
    k_data: torch.Tensor,
    v_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    output: torch.Tensor | None = None,
    *,
    page_size: int = 16,
    group_size: int = 32,
    softmax_scale: float | None = None,
    tokens_per_split: int = 0,
    waves_per_block: int = 0,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode attention that reads the packed INT4 paged cache directly.

    query [B, Hq, D] fp16; returns ``output`` (allocated with
    ``empty_like(query)`` when None).  Launch is asynchronous on the current
    stream.
    """
    if group_size != 32:
        raise NotImplementedError("decode fast path currently supports group_size=32")
    if k_data.ndim != 4 or tuple(v_data.shape) != tuple(k_data.shape):
        raise ValueError("k_data/v_data must have identical rank-4 shapes")
    num_pages, cache_page_size, num_kv_heads, packed_dim = k_data.shape
    _, _, head_dim = query.shape
    if cache_page_size != page_size or packed_dim * 2 != head_dim:
        raise ValueError("packed cache shape does not match query/page_size")
    batch, num_q_heads, head_dim, total, longest, block_table, seq_lens = _validate_common_decode_inputs(
        query, block_table, seq_lens, num_pages=num_pages, num_kv_heads=num_kv_heads,
        page_size=page_size, int4=True)
    scale_shape = (num_pages, page_size, num_kv_heads, head_dim // group_size)
    if tuple(k_scale.shape) != scale_shape:
        raise ValueError(f"k_scale must have shape {scale_shape}")
    if tuple(v_scale.shape) != scale_shape:
        raise ValueError(f"v_scale must have shape {scale_shape}")
    if k_data.dtype != torch.uint8 or v_data.dtype != torch.uint8:
        raise TypeError("k_data/v_data must use UINT8(torch.uint8)")
    if k_scale.dtype != torch.float16 or v_scale.dtype != torch.float16:
        raise TypeError("k_scale/v_scale must use FP16(torch.float16)")
    device = query.device
    for name, tensor in (("k_data", k_data), ("v_data", v_data), ("k_scale", k_scale),
                         ("v_scale", v_scale)):
        if tensor.device != device:
            raise ValueError(f"{name} must be on {device}")
    if output is None:
        output = torch.empty_like(query)
    elif output.shape != query.shape or output.dtype not in (query.dtype, torch.float32):
        raise ValueError("output must match query shape and dtype")
    elif output.device != query.device:
        raise ValueError("output must be on the same device as query")
    if batch == 0:
        return output
    scale = _qk_scale(head_dim, softmax_scale)
    plan = int4_decode_plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, block_table.shape[1],
                            total, longest, tokens_per_split, waves_per_block)
    _launch_decode(_dense(query, 16), k_data, v_data, k_scale, v_scale, block_table, seq_lens, output,
                   scale, plan, workspace)
    return output


def _int4_paged_decode_attention(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens,
                                 output, head_dim: int, page_size: int, group_size: int = 32,
                                 block_h: int = 16, block_n: int = 32, threads: int = 128,
                                 softmax_scale: float = 0.0) -> None:
    """Positional kernel handle with the reference's call shape
    (fused_attention.py:11-28).  No validation and no host synchronisation
    (the split plan uses block_table's width), so it can be captured in a
    HIP graph.  ``softmax_scale == 0.0`` means head_dim ** -0.5, as in the
    reference; block_h / block_n / threads are accepted and ignored."""
    del group_size, block_h, block_n, threads
    batch, num_q_heads, _ = query.shape
    if batch == 0:
        return
    scale = _qk_scale(head_dim, softmax_scale)
    plan = int4_decode_plan(batch, num_q_heads, k_data.shape[2], head_dim, k_data.shape[1],
                            block_table.shape[1])
    _launch_decode(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, scale,
                   plan)


# ---------------------------------------------------------------- FP16 cache


def fp16_decode_plan(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_pages: int,
                     total_tokens: int = -1, max_tokens: int = -1,
                     tokens_per_split: int = 0) -> tuple[int, int, int]:
    """(chunk_pages, max_chunks, workspace_bytes) from iris_fp16_decode_plan.

    A negative ``chunk_pages`` is the page-streaming kernel's plan; a negative
    ``tokens_per_split`` asks for that kernel (chunks of -tokens_per_split
    tokens), as A/B runs and tests do."""
    cp, mc = ctypes.c_int32(), ctypes.c_int32()
    ws = ctypes.c_int64()
    status = _lib.lib().iris_fp16_decode_plan(batch, num_q_heads, num_kv_heads, head_dim, max_pages,
                                              total_tokens, max_tokens, tokens_per_split,
                                              ctypes.byref(cp), ctypes.byref(mc), ctypes.byref(ws))
    _lib.check(status, "iris_fp16_decode_plan")
    return cp.value, mc.value, ws.value


def _launch_fp16_decode(query, k_cache, v_cache, block_table, seq_lens, output, softmax_scale: float,
                        plan, workspace=None) -> None:
    chunk_pages, max_chunks, ws_bytes = plan
    batch, num_q_heads, head_dim = query.shape
    num_pages, page_size, num_kv_heads, _ = k_cache.shape
    if ws_bytes > 0:
        workspace = _ready_workspace(query.device, ws_bytes, batch, workspace)
        ws_ptr, ws_len = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    else:
        ws_ptr, ws_len = 0, 0
    for name, t, align in (("query", query, 16), ("k_cache", k_cache, 16), ("v_cache", v_cache, 16),
                           ("block_table", block_table, 4), ("seq_lens", seq_lens, 4),
                           ("output", output, 4)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if t.data_ptr() % align:
            raise ValueError(f"{name} must be {align}-byte aligned")
    stream = _lib.raw_stream(query.device)
    status = _lib.lib().iris_fp16_paged_decode_attention(
        query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
        seq_lens.data_ptr(), output.data_ptr(), 1 if output.dtype == torch.float32 else 0, ws_ptr, ws_len,
        batch, num_q_heads, num_kv_heads, head_dim, page_size, num_pages, block_table.shape[1],
        float(softmax_scale), chunk_pages, max_chunks, stream)
    _lib.check(status, "iris_fp16_paged_decode_attention")


def fused_fp16_paged_decode_attention(
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    output: torch.Tensor | None = None,
    *,
    page_size: int = 16,
    softmax_scale: float | None = None,
    tokens_per_split: int = 0,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode attention over an fp16 paged cache [NP, page_size, Hkv, D]
    (the reference's matched baseline, fused_attention.py:528-582): same
    checks in the same order, same exception types and messages.  Returns
    ``output`` (allocated with ``empty_like(query)`` when None)."""
    if k_cache.ndim != 4 or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError("k_cache/v_cache must have identical rank-4 shapes")
    num_pages, cache_page_size, num_kv_heads, cache_dim = k_cache.shape
    _, _, head_dim = query.shape
    if cache_page_size != page_size or cache_dim != head_dim:
        raise ValueError("FP16 cache shape does not match query/page_size")
    batch, num_q_heads, head_dim, total, longest, block_table, seq_lens = _validate_common_decode_inputs(
        query, block_table, seq_lens, num_pages=num_pages, num_kv_heads=num_kv_heads,
        page_size=page_size)
    if k_cache.dtype != torch.float16 or v_cache.dtype != torch.float16:
        raise TypeError("k_cache/v_cache must use FP16")
    if k_cache.device != query.device or v_cache.device != query.device:
        raise ValueError("k_cache/v_cache must be on the query device")
    if output is None:
        output = torch.empty_like(query)
    elif output.shape != query.shape or output.dtype not in (query.dtype, torch.float32):
        raise ValueError("output must match query shape and dtype")
    elif output.device != query.device:
        raise ValueError("output must be on the same device as query")
    if batch == 0:
        return output
    scale = _qk_scale(head_dim, softmax_scale)
    plan = fp16_decode_plan(batch, num_q_heads, num_kv_heads, head_dim, block_table.shape[1], total,
                            longest, tokens_per_split)
    _launch_fp16_decode(_dense(query, 16), k_cache, v_cache, block_table, seq_lens, output, scale, plan,
                        workspace)
    return output


def _fp16_paged_decode_attention(query, k_cache, v_cache, block_table, seq_lens, output, head_dim: int,
                                 page_size: int, block_h: int = 16, block_n: int = 32, threads: int = 128,
                                 softmax_scale: float = 0.0) -> None:
    """Positional kernel handle with the reference's call shape
    (fused_attention.py:223-236): no validation and no host synchronisation
    (the split plan uses block_table's width).  ``softmax_scale == 0.0``
    means head_dim ** -0.5; block_h / block_n / threads are accepted and
    ignored."""
    del block_h, block_n, threads
    batch, num_q_heads, _ = query.shape
    if batch == 0:
        return
    num_kv_heads = k_cache.shape[2]
    plan = fp16_decode_plan(batch, num_q_heads, num_kv_heads, head_dim, block_table.shape[1])
    scale = _qk_scale(head_dim, softmax_scale)
    _launch_fp16_decode(query, k_cache, v_cache, block_table, seq_lens, output, scale, plan)
