"""The C ABI library: it loads, exports every function include/iris_hip.h
declares, and its host-side logic (argument checks, split plan) behaves.
Nothing here launches a kernel, so it runs without a GPU."""
import ctypes
import re
from pathlib import Path

import pytest

from iris_kernel import _lib
from iris_kernel.fused_attention import DECODE_PAGE_KERNEL, decode_plan, fp16_decode_plan

HEADER = Path(__file__).resolve().parents[1] / "include" / "iris_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|void|const char\s*\*)\s+(iris_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    assert declared_functions() == sorted(["iris_rope_int4_paged_append", "iris_decode_plan",
                                           "iris_int4_paged_decode_attention",
                                           "iris_int4_paged_decode_attention_noalloc", "iris_version",
                                           "iris_fp16_decode_plan", "iris_fp16_paged_decode_attention",
                                           "iris_rope_fp16_paged_append", "iris_quantize_pack_int4",
                                          "iris_decode_check", "iris_append_check"])


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(_lib.exported_symbols()) == set(declared_functions())
    assert lib.iris_version() == 100


def test_append_rejects_unsupported_head_dim_before_launch():
    lib = _lib.lib()
    null = None
    for d in (80, 0, 576):  # a multiple of 32 up to 512
        st = lib.iris_rope_int4_paged_append(null, null, null, null, null, null, null, null, null,
                                             null, 4, 2, d, d, 16, 8, 16, null)
        assert st == 1
    for rot in (-2, 130, 63):  # negative, past head_dim, odd
        st = lib.iris_rope_int4_paged_append(null, null, null, null, null, null, null, null, null,
                                             null, 4, 2, 128, rot, 16, 8, 16, null)
        assert st == 1
    # zero tokens is a no-op that touches nothing
    assert lib.iris_rope_int4_paged_append(null, null, null, null, null, null, null, null, null,
                                           null, 0, 2, 128, 64, 16, 8, 16, null) == 0


def test_decode_rejects_unsupported_shapes_before_launch():
    lib = _lib.lib()
    null = None
    base = dict(B=2, Hq=8, Hkv=2, D=128, P=16, NP=8, maxP=4, ct=2, mc=1, nw=4)
    def call(**kw):
        a = {**base, **kw}
        return lib.iris_int4_paged_decode_attention(null, null, null, null, null, null, null, null, 0,
                                                    null, 0, a["B"], a["Hq"], a["Hkv"], a["D"], a["P"],
                                                    a["NP"], a["maxP"], ctypes.c_float(0.1), a["ct"],
                                                    a["mc"], a["nw"], null)
    assert call(P=24) == 1          # page_size must be a multiple of 16 up to 256 (without the any-shape bit)
    assert call(P=8) == 1
    assert call(P=272) == 1
    assert call(P=512) == 1
    assert call(D=512) == 1         # head_dim in {64, 96, 128, 160, 192, 224, 256} (without the any-shape bit)
    assert call(D=80) == 1
    # head_dim 96, 160, 192, 224: their own kernel, 12 waves at 96, 8 above
    assert call(D=96, nw=12, ct=12, mc=1) == 2              # valid: it gets as far as the launch
    assert call(D=224, nw=8, ct=8, mc=1) == 2
    assert call(D=96, P=48, nw=12, ct=12, mc=1) == 2        # pages of 16 m tokens
    assert call(D=96) == 1                                  # its wave count only (4 asked)
    assert call(D=160, nw=12, ct=12, mc=1) == 1
    assert call(D=96, nw=12, ct=385, mc=1) == 1             # a chunk holds at most 32 tiles a wave: 384 at 12
    assert call(D=192, nw=8, ct=257, mc=1) == 1             # ... 256 at 8
    assert call(D=192, nw=8, ct=256, mc=1) == 2
    assert call(D=96, nw=12, ct=1, mc=1) == 1               # chunks do not cover max_pages
    assert call(D=96, nw=12, ct=2, mc=2) == 3               # two chunks need a workspace
    assert call(D=96, nw=12 | 0x100, ct=12, mc=1) == 1      # no selection bit but the any-shape one
    assert call(D=96, P=24, nw=12, ct=12, mc=1) == 1        # page sizes of 16 m tokens only
    # the any-shape kernel: any page size, head_dim a multiple of 32 up to 512
    any_ = 4 | 0x400
    assert call(P=48, D=96, nw=any_, ct=6, mc=1) == 2      # valid: it gets as far as the launch
    assert call(P=0, nw=any_) == 1                          # page_size >= 1
    assert call(D=80, nw=any_) == 1                         # multiple of 32
    assert call(D=544, nw=any_) == 1                        # at most 512
    assert call(P=48, nw=any_, ct=2, mc=2) == 1             # chunks do not cover 4 x 48 tokens
    assert call(P=48, nw=any_, ct=3, mc=4) == 1             # chunks of whole 64-token tiles
    assert call(P=48, nw=any_, ct=2, mc=3) == 3             # three chunks need a workspace
    assert call(nw=0x400 | 0x100) == 1                      # one selection bit at most
    assert call(nw=0x800 | 0x400) == 1
    # the token-page mode: any page size, head_dim 64-224
    tok = 0x800
    assert call(D=96, P=24, nw=12 | tok, ct=12, mc=1) == 2   # valid: it gets as far as the launch
    assert call(D=64, P=1, nw=16 | tok, ct=16, mc=1) == 2
    assert call(D=128, P=8, nw=8 | tok, ct=8, mc=1) == 2
    assert call(D=224, P=16, nw=8 | tok, ct=8, mc=1) == 2   # 16-token pages too
    assert call(D=96, P=24, Hkv=1, nw=12 | tok, ct=12, mc=1) == 2  # 3 x 1 scale halves a row: odd
    assert call(D=96, P=3, NP=7, Hkv=1, nw=12 | tok, ct=12, mc=1) == 2  # ... in an odd pool: the any kernel
    assert call(D=96, P=3, NP=7, Hkv=1, nw=12 | tok, ct=3, mc=1) == 1   # (whose chunks are even tile counts)
    assert call(D=256, P=8, nw=8 | tok, ct=8, mc=1) == 2    # head_dim 64 to 256
    assert call(D=288, P=8, nw=8 | tok, ct=8, mc=1) == 1
    assert call(D=96, P=24, nw=8 | tok, ct=12, mc=1) == 1   # its wave count only
    assert call(D=96, P=0, nw=12 | tok, ct=12, mc=1) == 1   # page_size >= 1
    assert call(D=96, P=200, nw=12 | tok, ct=12, mc=2) == 1  # chunks do not cover 4 x 200 tokens
    assert call(D=96, P=200, nw=12 | tok, ct=24, mc=2) == 3  # two chunks need a workspace
    assert call(D=96, P=2, NP=(1 << 31) + 1, nw=12 | tok, ct=12, mc=1) == 1  # token slots in 32 bits
    assert call(Hq=9) == 1          # Hq not divisible by Hkv
    assert call(ct=1, mc=1) == 1    # chunks do not cover max_pages
    assert call(nw=5) == 1
    assert call(ct=1, mc=2) == 3    # two chunks need a workspace
    # 16 waves: the page-streaming kernel (Hkv=2, D=128 is one of its shapes)
    assert call(nw=16, ct=65, mc=1, maxP=4) == 1   # a chunk holds at most 64 tiles
    assert call(nw=16, ct=1, mc=1) == 1            # chunks do not cover max_pages
    assert call(nw=16, ct=1, mc=2) == 3            # two chunks need a workspace
    assert call(nw=16, Hkv=3, Hq=9) == 1           # Hkv=3 has no page-kernel layout


def test_fp16_and_write_side_entry_points_reject_bad_arguments_before_launch():
    lib = _lib.lib()
    null = None
    def dec(**kw):
        a = {**dict(B=2, Hq=8, Hkv=2, D=128, P=16, NP=8, maxP=4, cp=4, mc=1), **kw}
        return lib.iris_fp16_paged_decode_attention(null, null, null, null, null, null, 0, null, 0, a["B"],
                                                    a["Hq"], a["Hkv"], a["D"], a["P"], a["NP"], a["maxP"],
                                                    ctypes.c_float(0.1), a["cp"], a["mc"], null)
    assert dec(P=32) == 1           # page_size must be 16
    assert dec(D=96) == 1           # head_dim in {64, 128}
    assert dec(Hq=34, Hkv=2) == 1   # more than 16 query heads per kv head
    assert dec(cp=1, mc=1) == 1     # chunks do not cover max_pages
    assert dec(cp=257) == 1         # a chunk holds at most 256 pages
    assert dec(cp=2, mc=2) == 3     # two chunks need a workspace
    def app(T=4, H=2, D=64, rot=64, P=16):
        return lib.iris_rope_fp16_paged_append(null, null, null, null, null, null, null, null, T, H, D, rot, P,
                                               8, 16, null)
    assert app(rot=66) == 1         # rotary_dim > head_dim
    assert app(rot=3) == 1          # odd rotary_dim
    assert app(P=0) == 1
    assert app(T=0) == 0            # zero tokens: a no-op that touches nothing
    qp = lambda T, D: lib.iris_quantize_pack_int4(null, null, null, T, 2, D, null)
    assert qp(4, 96) == 1           # head_dim % 64
    assert qp(4, 576) == 1          # head_dim <= 512
    assert qp(0, 128) == 0


def test_fp16_decode_plan():
    # configuration 2's shape and lengths: the page-streaming kernel (negative
    # chunk_pages), chunks of all kv heads, one workgroup a CU
    cp, mc, ws = fp16_decode_plan(32, 32, 8, 128, 256, 32 * 4096, 4096)
    assert cp < 0 and -cp * mc >= 256 and -cp * (mc - 1) < 256 and -cp <= 128 and mc <= 16
    assert 32 * mc == 256 and ws > 0
    # ragged lengths: the per-kv-head kernel
    cp, mc, ws = fp16_decode_plan(32, 32, 8, 128, 256, 16 * 4096, 4096)
    assert cp > 0 and cp * mc >= 256 and cp * (mc - 1) < 256 and cp <= 256
    assert mc > 1 and ws > 0
    # one chunk when the longest sequence fits in one (here 4 pages < 8)
    cp, mc, ws = fp16_decode_plan(4, 8, 2, 64, 4, 200, 60)
    assert (cp, mc, ws) == (4, 1, 0)
    cp, mc, _ = fp16_decode_plan(2, 8, 2, 128, 64, tokens_per_split=64)
    assert (cp, mc) == (4, 16)
    with pytest.raises(RuntimeError):
        fp16_decode_plan(2, 8, 2, 96, 64)
    # the page-streaming kernel needs 8 sequences and 64 MB of K/V: one
    # sequence of 4096 tokens (17 MB) or four (67 MB) get the other kernel,
    # eight (134 MB) the page-streaming one
    assert fp16_decode_plan(1, 32, 8, 128, 256, 4096, 4096)[0] > 0
    assert fp16_decode_plan(4, 32, 8, 128, 256, 4 * 4096, 4096)[0] > 0
    assert fp16_decode_plan(8, 32, 8, 128, 256, 8 * 4096, 4096)[0] < 0
    assert fp16_decode_plan(8, 16, 8, 64, 256, 8 * 4096, 4096)[0] < 0      # 67 MB at head_dim 64
    # ... unless asked for with a negative tokens_per_split (chunks of that many tokens)
    cp, mc, ws = fp16_decode_plan(1, 32, 8, 128, 256, 4096, 4096, -1024)
    assert (cp, mc) == (-64, 4) and ws > 0
    assert fp16_decode_plan(1, 32, 8, 128, 256, 4096, 4096, -2048)[:2] == (-128, 2)   # 128-page chunks
    for bad in ((1, 32, 2, 128, 256, 4096, 4096, -1024),     # 2 kv heads: no page-streaming layout
                (1, 32, 8, 128, 256, 4096, 4096, -4096)):    # 256-page chunks
        with pytest.raises(RuntimeError):
            fp16_decode_plan(*bad)


def general_kvw(B, Hq, Hkv, max_pages):
    """KV heads per wave of the general kernel (decode.hip pick_kvw): the
    most that fit 16 MFMA columns and divide Hkv, halved while the grid
    would hold under 512 wave-tiles at the block table's capacity."""
    kvw = 4
    while kvw > 1 and (kvw * (Hq // Hkv) > 16 or Hkv % kvw):
        kvw //= 2
    cap_tiles = (max_pages * 16 + 31) // 32
    while kvw > 1 and B * (cap_tiles + 1) * (Hkv // kvw) < 512:
        kvw //= 2
    return kvw


def counter_bytes(B):
    """The arrival-counter region every decode kernel keeps at the head of its
    workspace: 128 uint32 per sequence (IRIS_COUNTER_BYTES)."""
    return (B * 128 * 4 + 255) // 256 * 256


def general_workspace(B, Hq, Hkv, D, max_chunks, max_pages):
    """Workspace bytes of the general kernel's split (decode.hip)."""
    n_kvb = Hkv // general_kvw(B, Hq, Hkv, max_pages)
    return counter_bytes(B) + B * max_chunks * n_kvb * 16 * (D + 2) * 4


def pages_workspace(B, Hq, D, max_chunks, balanced=False):
    """Workspace bytes of the page kernel's split (decode_pages.hip): one slot
    per (workgroup, sequence) pair a workgroup can work on (workgroups + B:
    B x max_chunks workgroups in chunk mode, max_chunks in the balanced
    mode); the counter region, chunk partials, and group partials when a
    sequence can span more than one group of 8 chunks."""
    r = lambda x: (x + 255) // 256 * 256  # noqa: E731
    slots = (max_chunks if balanced else B * max_chunks) + B
    s2 = slots if max_chunks > 8 else 0
    return (counter_bytes(B) + r(slots * Hq * D * 4) + r(slots * Hq * 2 * 4)
            + r(s2 * Hq * D * 4) + r(s2 * Hq * 2 * 4))


@pytest.mark.parametrize("cfg,expect_chunks,kernel", [
    # (B, Hq, Hkv, D, maxP, total, max)
    ((32, 32, 8, 128, 256, 32 * 4096, 4096), True, "pages"),      # Llama-3-8B shape: page kernel
    ((64, 32, 8, 128, 1024, 64 * 3000, 16384), True, "pages"),    # ragged batch: page kernel, balanced mode
    ((4, 64, 8, 128, 8192, 4 * 131072, 131072), True, "pages"),   # 8 query heads per kv head: streaming kernel
    ((4, 8, 2, 64, 16, 400, 200), False, "general"),              # D = 64: general; tiny grid, one chunk
    ((8, 32, 8, 128, 512, 8 * 8192, 8192), True, "hd"),           # 75 MB of K/V: head-dim kernel, token pages
    ((64, 32, 8, 128, 64, 64 * 1024, 1024), True, "general"),     # 512 units: general kernel
    ((64, 32, 8, 128, 256, 64 * 1000, 4096), True, "general"),    # ragged: general kernel
])
def test_decode_plan_covers_every_tile(cfg, expect_chunks, kernel):
    B, Hq, Hkv, D, maxP, total, mx = cfg
    chunk_tiles, max_chunks, nw, ws = decode_plan(B, Hq, Hkv, D, maxP, total, mx)
    if chunk_tiles < 0:  # the balanced mode (test_balanced_plan_for_ragged_lengths)
        assert kernel == "pages" and nw == 16 and -chunk_tiles <= 64
        assert ws == pages_workspace(B, Hq, D, max_chunks, balanced=True)
        return
    tiles = (maxP * 16 + 31) // 32
    assert chunk_tiles * max_chunks >= tiles
    assert (chunk_tiles * (max_chunks - 1)) < tiles
    assert (max_chunks > 1) == expect_chunks
    if kernel == "hd":
        w = 16 if D == 64 else 8
        assert nw == w | 0x800 and chunk_tiles % w == 0 and chunk_tiles <= 32 * w
        assert ws == (any_workspace(B, Hq, D, max_chunks) if max_chunks > 1 else 0)
        return
    assert (nw == 16) == (kernel == "pages") and (nw == 16 or 1 <= nw <= 4)
    assert chunk_tiles <= 64  # a chunk's page ids fit two VGPRs
    if max_chunks == 1:
        assert ws == 0
    elif nw == 16:
        assert ws == pages_workspace(B, Hq, D, max_chunks)
    else:
        assert ws == general_workspace(B, Hq, Hkv, D, max_chunks, maxP)


def test_gqa8_plans():
    # 8 query heads per kv head (D=128, Hkv=8): the streaming kernel has a
    # chunk mode only, so 16-wave requests get chunk plans even for ragged
    # lengths; the page-kernel bit keeps the page kernel's balanced mode; a
    # block table wider than 64 chunks of 64 tiles leaves the plan's choice to
    # the general kernel; a short batch goes to the head-dim kernel's
    # token-page mode (at head_dim 64 only from 4 MB of K/V; never with one
    # kv head).
    B, Hq, Hkv, D = 4, 64, 8, 128
    ct, mc, nw, ws = decode_plan(B, Hq, Hkv, D, 8192, B * 131072, 131072)
    assert (ct, mc, nw) == (64, 64, 16) and ws == pages_workspace(B, Hq, D, 64)
    ct, mc, nw, _ = decode_plan(B, Hq, Hkv, D, 8192, 131072 + 3 * 5000, 131072, waves_per_block=16)
    assert ct > 0 and mc <= 64 and nw == 16
    ct, mc, nw, _ = decode_plan(B, Hq, Hkv, D, 8192, 131072 + 3 * 5000, 131072,
                                waves_per_block=16 | DECODE_PAGE_KERNEL)
    assert ct < 0 and nw == 16 | DECODE_PAGE_KERNEL
    assert decode_plan(B, Hq, Hkv, D, 8193, B * 131072, 131072)[2] <= 4
    assert decode_plan(1, Hq, Hkv, D, 8192, 131072, 131072)[2] <= 4   # one or two sequences: the general kernel
    assert decode_plan(2, Hq, Hkv, D, 8192, 2 * 131072, 131072)[2] <= 4
    assert decode_plan(3, Hq, Hkv, D, 4096, 3 * 65536, 65536)[2] == 16
    assert decode_plan(B, Hq, Hkv, D, 64, B * 1024, 1024)[2] == 8 | 0x800  # the head-dim kernel
    assert decode_plan(B, Hq, Hkv, D, 64, B * 512, 512)[2] == 8 | 0x800
    assert decode_plan(B, 32, 8, 64, 64, B * 512, 512)[2] <= 4              # head_dim 64, 1.2 MB: general
    assert decode_plan(B, 32, 8, 64, 256, B * 4096, 4096)[2] == 16 | 0x800  # head_dim 64, 9.4 MB
    assert decode_plan(1, 16, 1, 128, 1024, 16384, 16384)[2] <= 4           # one kv head: general


@pytest.mark.parametrize("cfg", [
    # (B, Hq, Hkv, D, maxP, total, max): ragged lengths known, page kernel asked for
    (64, 32, 8, 128, 1024, 64 * 3000, 16384),
    (3, 32, 8, 128, 1024, 16384 + 200 + 17, 16384),
    (200, 16, 4, 128, 64, 200 * 500, 1024),
])
def test_balanced_plan_for_ragged_lengths(cfg):
    B, Hq, Hkv, D, maxP, total, mx = cfg
    share, wgs, nw, ws = decode_plan(B, Hq, Hkv, D, maxP, total, mx, waves_per_block=16)
    assert nw == 16 and share < 0  # negative: the balanced mode
    tiles_ub = (total + 31) // 32 + B
    assert 1 <= -share <= 64 and -share * wgs >= tiles_ub  # every share within the page-id window
    assert wgs <= 512
    assert ws == (pages_workspace(B, Hq, D, wgs, balanced=True) if wgs > 1 else 0)
    # uniform lengths keep chunk mode
    assert decode_plan(B, Hq, Hkv, D, maxP, B * mx, mx, waves_per_block=16)[0] > 0


def test_decode_plan_overrides_and_errors():
    ct, mc, nw, ws = decode_plan(2, 8, 2, 128, 64, tokens_per_split=64, waves_per_block=2)
    assert (ct, mc, nw) == (2, 16, 2)
    assert ws == general_workspace(2, 8, 2, 128, 16, 64)
    # 16 waves forces the page kernel on a shape it supports but would not pick
    ct, mc, nw, ws = decode_plan(2, 8, 2, 128, 64, tokens_per_split=64, waves_per_block=16)
    assert (ct, mc, nw) == (2, 16, 16)
    assert ws == pages_workspace(2, 8, 128, 16)
    # ... and falls back to the general kernel where it has no layout (Hkv=3)
    assert decode_plan(2, 9, 3, 128, 64, waves_per_block=16)[2] == 4
    # head_dim 96, 160, 192, 224 plan their own kernel: chunks of whole steps
    # of its waves (256 tokens -> 8 tiles -> 12 at 12 waves), the any-shape
    # kernel's workspace layout
    ct, mc, nw, ws = decode_plan(2, 8, 2, 96, 64, tokens_per_split=256)
    assert (ct, mc, nw) == (12, 3, 12), (ct, mc, nw)
    assert ws == any_workspace(2, 8, 96, 3)
    ct, mc, nw, ws = decode_plan(2, 40, 2, 224, 64, tokens_per_split=256)
    assert (ct, mc, nw) == (8, 4, 8), (ct, mc, nw)
    assert ws == any_workspace(2, 40, 224, 4)
    assert decode_plan(1, 8, 8, 160, 64)[:3] == (8, 4, 8)   # 32 tiles over 8 units: a tile a wave
    assert decode_plan(4, 32, 8, 192, 4096)[2] == 8
    # ... and the any-shape kernel when asked; other head dims plan it by themselves
    ct, mc, nw, ws = decode_plan(2, 8, 2, 96, 64, tokens_per_split=256, waves_per_block=0x400)
    assert (ct, mc, nw) == (8, 4, 4 | 0x400), (ct, mc, nw)
    assert ws == any_workspace(2, 8, 96, 4)
    assert decode_plan(2, 8, 2, 512, 64)[2] == 4 | 0x400
    assert decode_plan(2, 8, 2, 32, 64)[2] == 4 | 0x400
    for bad in (80, 544, 0):
        with pytest.raises(RuntimeError):
            decode_plan(2, 8, 2, bad, 64)
    # the token-page mode when asked: the head-dim kernel's waves (16 at 64,
    # 12 at 96, 8 above) and its workspace layout; the any-shape kernel's
    # plan where it does not take the shape
    assert decode_plan(2, 8, 2, 128, 64, waves_per_block=0x800)[2] == 8 | 0x800
    assert decode_plan(2, 8, 2, 64, 64, waves_per_block=0x800)[2] == 16 | 0x800
    assert decode_plan(2, 8, 1, 64, 64, waves_per_block=0x800)[2] == 16 | 0x800
    assert decode_plan(2, 8, 2, 96, 64, waves_per_block=0x800)[2] == 12 | 0x800
    assert decode_plan(2, 8, 1, 96, 64, waves_per_block=0x800)[2] == 12 | 0x800  # 3 halves a row
    assert decode_plan(2, 8, 2, 256, 64, waves_per_block=0x800)[2] == 8 | 0x800
    assert decode_plan(2, 8, 2, 256, 64)[2] == 8 | 0x800                        # the plan's own choice
    assert decode_plan(2, 8, 1, 256, 64)[2] <= 4                                # one kv head: general
    assert decode_plan(2, 8, 2, 256, 64, waves_per_block=4)[2] == 4
    assert decode_plan(2, 8, 2, 288, 64, waves_per_block=0x800)[2] == 4 | 0x400
    ct, mc, nw, ws = decode_plan(2, 8, 2, 160, 64, tokens_per_split=256, waves_per_block=0x800)
    assert (ct, mc, nw) == (8, 4, 8 | 0x800), (ct, mc, nw)
    assert ws == any_workspace(2, 8, 160, 4)
    # page sizes that are not a multiple of 16 up to 256: int4_decode_plan
    # asks for the token-page mode (the any-shape kernel where that does
    # not take the shape, or when the caller asks for it); multiples of 16
    # (48, 80, ...) plan the fast kernels over 16-token pages
    from iris_kernel.fused_attention import int4_decode_plan

    assert int4_decode_plan(2, 8, 2, 128, 24, 10)[2] == 8 | 0x800
    assert int4_decode_plan(2, 8, 2, 128, 1, 1000)[2] == 8 | 0x800
    assert int4_decode_plan(2, 8, 2, 128, 272, 10)[2] == 8 | 0x800
    assert int4_decode_plan(2, 8, 1, 96, 24, 10)[2] == 12 | 0x800
    assert int4_decode_plan(2, 8, 1, 256, 24, 10)[2] == 8 | 0x800
    assert int4_decode_plan(2, 8, 2, 256, 24, 10)[2] == 8 | 0x800
    assert int4_decode_plan(2, 8, 2, 288, 24, 10)[2] == 4 | 0x400
    assert int4_decode_plan(2, 8, 2, 128, 24, 10, waves_per_block=0x400)[2] == 4 | 0x400
    assert int4_decode_plan(2, 8, 2, 128, 32, 10)[2] in (4, 16, 8 | 0x800)
    assert int4_decode_plan(2, 8, 2, 128, 48, 10)[2] in (1, 2, 3, 4, 16, 8 | 0x800)
    assert int4_decode_plan(2, 8, 2, 128, 32, 10, waves_per_block=4)[2] == 4
    ct, mc, nw, ws = int4_decode_plan(3, 8, 2, 128, 8, 60, tokens_per_split=64)
    assert ct * 32 * mc >= 60 * 8 and ct % 8 == 0 and nw == 8 | 0x800
    ct, mc, nw, ws = int4_decode_plan(3, 8, 2, 128, 8, 60, tokens_per_split=64, waves_per_block=0x400)
    assert ct * 32 * mc >= 60 * 8 and ct % 2 == 0 and nw & 0x400


def any_workspace(batch, hq, d, max_chunks):
    """Split-KV workspace of the any-shape kernel: counters, then o / l
    [B][chunks][Hq][D] and (m, l) [B][chunks][Hq][2] fp32."""
    up = lambda x: (x + 255) // 256 * 256
    return up(batch * 512) + up(batch * max_chunks * hq * d * 4) + batch * max_chunks * hq * 2 * 4


def test_decode_check_rejects_bad_arguments_before_launch():
    lib = _lib.lib()
    state = ctypes.c_void_p(16)  # never dereferenced: each call fails its argument checks first
    assert lib.iris_decode_check(None, None, 1, 4, 10, 16, None, None, None) == 1       # no state
    assert lib.iris_decode_check(None, None, 1, 4, 10, 16, state, None, None) == 1      # no seq_lens
    assert lib.iris_decode_check(state, None, 1, 4, 10, 16, state, None, None) == 1     # no block_table
    assert lib.iris_decode_check(state, state, 1, 4, 10, 0, state, None, None) == 1     # page_size 0
    assert lib.iris_decode_check(state, state, -1, 4, 10, 16, state, None, None) == 1   # negative batch
    assert lib.iris_decode_check(state, state, 2, 1 << 62, 10, 16, state, None, None) == 1  # table too large


def test_append_check_rejects_bad_arguments_before_launch():
    lib = _lib.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: each call fails its argument checks first
    assert lib.iris_append_check(p, p, 4, 64, 10, None, p, 2, None, None) == 1   # no state
    assert lib.iris_append_check(None, p, 4, 64, 10, p, p, 2, None, None) == 1   # no slot_mapping
    assert lib.iris_append_check(p, None, 4, 64, 10, p, p, 2, None, None) == 1   # no positions
    assert lib.iris_append_check(p, p, 4, 65, 10, p, p, 2, None, None) == 1      # bitmap too small
    assert lib.iris_append_check(p, p, -1, 64, 10, p, p, 2, None, None) == 1     # negative count


def test_decode_kernel_selection_bits(monkeypatch):
    # The kernel a plan names travels in its wave count (selection bits
    # above the low byte); nothing in the environment changes it.
    from iris_kernel.fused_attention import DECODE_PAGE_KERNEL, DECODE_VALU_TILE

    shape = (32, 32, 8, 128, 256, 32 * 4096, 4096)
    assert decode_plan(*shape)[2] == 16
    monkeypatch.setenv("IRIS_DECODE_KERNEL", "general")  # the retired switch is ignored
    assert decode_plan(*shape)[2] == 16
    assert decode_plan(*shape, waves_per_block=4)[2] == 4
    assert decode_plan(*shape, waves_per_block=16 | DECODE_PAGE_KERNEL)[2] == 16 | DECODE_PAGE_KERNEL
    assert decode_plan(*shape, waves_per_block=DECODE_VALU_TILE)[2] == 4 | DECODE_VALU_TILE
    assert decode_plan(*shape, waves_per_block=16 | DECODE_VALU_TILE)[2] == 4 | DECODE_VALU_TILE
    # MQA shape: a 16-wave plan runs the MQA kernel unless the page kernel is asked for
    mqa = (128, 16, 1, 64, 512, 128 * 8192, 8192)
    assert decode_plan(*mqa)[2] == 16
    assert decode_plan(*mqa, waves_per_block=DECODE_PAGE_KERNEL)[2] in (16 | DECODE_PAGE_KERNEL, 4)
    with pytest.raises(RuntimeError):
        decode_plan(*shape, waves_per_block=DECODE_PAGE_KERNEL | DECODE_VALU_TILE)
    with pytest.raises(RuntimeError):
        decode_plan(*shape, waves_per_block=0x1000)
    with pytest.raises(RuntimeError):
        decode_plan(*shape, waves_per_block=0x800 | 0x400)


def test_valu_tile_selection_covers_two_layouts():
    # The VALU bit plans the general kernel and runs its VALU tile for g = 4
    # at D = 128 (four kv heads a wave) and g = 16 at D = 64; every other
    # shape is refused before any HIP call (null pointers are safe).  The
    # page-kernel bit on a general-kernel wave count is refused too.
    from iris_kernel.fused_attention import DECODE_PAGE_KERNEL, DECODE_VALU_TILE

    lib = _lib.lib()
    null = None
    def call(B, Hq, Hkv, D, maxP, waves=4 | DECODE_VALU_TILE):
        return lib.iris_int4_paged_decode_attention(null, null, null, null, null, null, null, null, 0,
                                                    null, 0, B, Hq, Hkv, D, 16, 8, maxP, ctypes.c_float(0.1),
                                                    64, (maxP + 127) // 128, waves, null)
    assert call(2, 8, 2, 64, 4) == 1       # g = 4 at D = 64
    assert call(2, 8, 2, 128, 4) == 1      # g = 4 at D = 128, but two kv heads a wave
    assert call(2, 16, 2, 128, 4) == 1     # g = 8
    assert call(2, 16, 1, 256, 4) == 1     # D = 256
    assert call(2, 16, 4, 128, 4) == 1     # g = 4, Hkv = 4: one kv head a wave at this size
    assert call(2, 16, 4, 128, 4, 4 | DECODE_PAGE_KERNEL) == 1
    assert call(2, 16, 4, 128, 4, 4 | DECODE_PAGE_KERNEL | DECODE_VALU_TILE) == 1


def test_fused_api_requires_a_gpu_when_none_is_present():
    import torch

    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from iris_kernel.fused_attention import fused_int4_paged_decode_attention
    from iris_kernel.fused_kv import fused_rope_int4_paged_append

    x = torch.zeros(1, 1, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="require CUDA"):
        fused_rope_int4_paged_append(x, x, torch.zeros(1, dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
                                     torch.zeros(1, 32, dtype=torch.float16), torch.zeros(1, 32, dtype=torch.float16),
                                     torch.zeros(1, 16, 1, 32, dtype=torch.uint8), torch.zeros(1, 16, 1, 32, dtype=torch.uint8),
                                     torch.zeros(1, 16, 1, 2, dtype=torch.float16), torch.zeros(1, 16, 1, 2, dtype=torch.float16),
                                     rotary_dim=64, page_size=16)
    with pytest.raises(RuntimeError, match="require CUDA"):
        fused_int4_paged_decode_attention(x, torch.zeros(1, 16, 1, 32, dtype=torch.uint8),
                                          torch.zeros(1, 16, 1, 32, dtype=torch.uint8),
                                          torch.zeros(1, 16, 1, 2, dtype=torch.float16),
                                          torch.zeros(1, 16, 1, 2, dtype=torch.float16),
                                          torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32))
