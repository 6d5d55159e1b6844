"""INT4 decode over pages of any size on the token-page mode of the
head-dim MFMA kernel (csrc/decode_hd.hip, IRIS_DECODE_TOKEN_PAGES): each of
a tile's 32 tokens finds its page through the block table, so the page size
is free (the reference's eager path takes any page size,
torch_eager_attention.py:72; its fused path only 16, fused_attention.py:
390-403).  Head dims 64 to 256 in steps of 32, any number of kv heads (where
head_dim / 32 x num_kv_heads is odd, a kv head's scales start on either
half of a dword, by the token's slot, and the shift is taken per token).  Checked against the checker's eager attention
(fp32 values within helpers.ATOL; fp16 outputs within one ulp), with one
chunk a sequence and with split-KV, against the any-shape kernel, on caches
written by the package's own append, through the positional handle and in
a HIP graph."""
import pytest
import torch

from helpers import assert_attention_close, log, to
from iris_kernel import workloads
from iris_kernel.fused_attention import (DECODE_ANY_KERNEL, DECODE_TOKEN_PAGES, _int4_paged_decode_attention,
                                         fused_int4_paged_decode_attention, int4_decode_plan)
from iris_kernel.fused_kv import fused_rope_int4_paged_append
from oracle.torch_eager_attention import torch_eager_int4_paged_decode_attention
from oracle.torch_eager_kv import pack_int4, quantize_int4_groupwise

pytestmark = pytest.mark.gpu


def _waves(d):
    return 16 if d == 64 else 12 if d == 96 else 8


def _case(hq, hkv, d, page, lens, seed, spare=3):
    """A paged INT4 pool of random fp16 K/V quantised as the append writes
    it, a shuffled block table wide enough for the longest sequence (one
    spare column), and a query."""
    g = torch.Generator().manual_seed(seed)
    cols = -(-max(lens) // page) + 1
    n_pages = len(lens) * cols + spare
    pool = []
    for _ in range(2):
        x = (torch.randn(n_pages, page, hkv, d, generator=g) * 1.5).to(torch.float16)
        codes, scales = quantize_int4_groupwise(x, 32)
        pool.append((pack_int4(codes), scales))
    (kd, ks), (vd, vs) = pool
    bt = torch.randperm(n_pages, generator=g)[: len(lens) * cols].view(len(lens), cols).to(torch.int32)
    q = torch.randn(len(lens), hq, d, generator=g).to(torch.float16)
    return q, (kd, vd, ks, vs), bt, torch.tensor(lens, dtype=torch.int32)


def _check(device, q, cache, bt, sl, page, what, **kw):
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=page, out_dtype=torch.float32)
    gq, gbt, gsl = to(device, q, bt, sl)
    gcache = to(device, *cache)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(gq, *gcache, gbt, gsl, out, page_size=page, **kw)
    torch.cuda.synchronize(device)
    e32 = assert_attention_close(out, want, f"{what} fp32")
    out16 = fused_int4_paged_decode_attention(gq, *gcache, gbt, gsl, page_size=page, **kw)
    torch.cuda.synchronize(device)
    e16 = assert_attention_close(out16, want.to(torch.float16), f"{what} fp16")
    return out, e32, e16


@pytest.mark.parametrize("tps", [0, 128])
@pytest.mark.parametrize("hq,hkv,d,page,lens", [
    (8, 2, 128, 8, [1, 17, 300, 1000]),           # 8-token pages, head_dim 128
    (16, 1, 64, 1, [1, 33, 500]),                 # one token a page, MQA at head_dim 64
    (12, 3, 64, 24, [31, 32, 33, 1200]),          # 3 kv heads (2 groups each: whole dwords)
    (8, 2, 96, 24, [47, 48, 49, 2000]),           # head_dim 96
    (16, 2, 160, 40, [100, 2000]),                # head_dim 160
    (32, 8, 192, 3, [64, 65, 777]),               # 3-token pages, head_dim 192
    (28, 4, 224, 100, [5, 31, 33, 1500]),         # head_dim 224, 7 query heads per kv head
    (40, 2, 96, 8, [77, 1234]),                   # 20 query heads per kv head: two blocks
    (64, 1, 128, 12, [500, 3]),                   # 64 query heads on one kv head: four blocks
    (6, 3, 128, 5, [1, 79, 81, 3000]),            # 3 kv heads at head_dim 128
    (16, 4, 128, 300, [1000, 4000]),              # 300-token pages
    (16, 2, 224, 16, [16, 32, 48, 900]),          # 16-token pages, asked for
    (16, 2, 256, 8, [1, 300, 1000]),              # head_dim 256
    (12, 3, 256, 24, [47, 1500]),                 # head_dim 256, 3 kv heads
    (32, 8, 256, 16, [64, 2000]),                 # head_dim 256, 16-token pages (the plan's own choice)
])
def test_token_pages_match_eager(device, hq, hkv, d, page, lens, tps):
    log(f"decode tok: Hq={hq} Hkv={hkv} D={d} P={page} lens={lens} split={tps}")
    q, cache, bt, sl = _case(hq, hkv, d, page, lens, hq * 7 + d + page + tps)
    kw = {"waves_per_block": DECODE_TOKEN_PAGES} if page % 16 == 0 and page <= 256 else {}
    plan = int4_decode_plan(len(lens), hq, hkv, d, page, bt.shape[1], int(sl.sum()), int(sl.max()), tps,
                            kw.get("waves_per_block", 0))
    assert plan[2] == _waves(d) | DECODE_TOKEN_PAGES, plan
    _, e32, e16 = _check(device, q, cache, bt, sl, page, f"Hq={hq} Hkv={hkv} D={d} P={page} split={tps}",
                         tokens_per_split=tps, **kw)
    log(f"decode tok: max-abs err fp32 {e32:.2e} fp16 {e16:.2e} (plan {plan})")


@pytest.mark.parametrize("d,page", [(64, 8), (96, 24), (128, 1), (160, 40), (192, 8), (224, 3), (256, 12)])
def test_token_pages_agree_with_the_any_kernel(device, d, page):
    # The two kernels that serve these page sizes, on one case with many
    # chunks: within the same bound of each other as of the eager result.
    q, cache, bt, sl = _case(8, 2, d, page, [2500, 129, 1800], d + page)
    out, _, _ = _check(device, q, cache, bt, sl, page, f"tok D={d} P={page}", tokens_per_split=256)
    ref, _, _ = _check(device, q, cache, bt, sl, page, f"any D={d} P={page}", tokens_per_split=256,
                       waves_per_block=DECODE_ANY_KERNEL)
    e = assert_attention_close(out, ref, f"tok against any D={d} P={page}")
    log(f"decode tok: D={d} P={page} against the any kernel {e:.2e}")


@pytest.mark.parametrize("tps", [0, 128])
@pytest.mark.parametrize("hq,hkv,d,page,lens", [
    (8, 1, 96, 24, [300, 1000]),                  # 3 scale halves a token row
    (9, 3, 96, 8, [1, 33, 700]),                  # 9
    (5, 5, 160, 12, [100, 1500]),                 # 25
    (7, 1, 224, 40, [41, 2000]),                  # 7
    (16, 1, 96, 1, [1, 2, 31, 500]),              # one token a page
    (3, 3, 160, 16, [16, 47, 900]),               # 16-token pages, asked for
])
def test_odd_scale_rows(device, hq, hkv, d, page, lens, tps):
    # head_dim / 32 x Hkv odd: a kv head's scales start on either half of a
    # dword, by the token's slot; the mode takes the shift per token.  In a
    # pool of an even number of token slots the token-page mode runs; in an
    # odd one (the scale tensors end on half a dword) the launch takes the
    # any-shape kernel with the same plan.
    kw = {"waves_per_block": DECODE_TOKEN_PAGES} if page % 16 == 0 else {}
    for spare in (2, 3):
        q, cache, bt, sl = _case(hq, hkv, d, page, lens, hq + d + page + spare + tps, spare=spare)
        slots = cache[0].shape[0] * page
        plan = int4_decode_plan(len(lens), hq, hkv, d, page, bt.shape[1], int(sl.sum()), int(sl.max()), tps,
                                kw.get("waves_per_block", 0))
        assert plan[2] == _waves(d) | DECODE_TOKEN_PAGES, plan
        what = f"odd rows Hq={hq} Hkv={hkv} D={d} P={page} slots={slots} split={tps}"
        log(f"decode tok: {what}")
        _, e32, e16 = _check(device, q, cache, bt, sl, page, what, tokens_per_split=tps, **kw)
        log(f"decode tok: {what}: fp32 {e32:.2e} fp16 {e16:.2e}")


@pytest.mark.parametrize("d,page,hkv", [(128, 8, 2), (96, 24, 4), (224, 40, 2), (64, 1, 1)])
def test_token_pages_read_what_the_append_writes(device, d, page, hkv):
    # A cache the package's own append wrote, read back by the decode: the
    # two ends of the path at the same shapes.
    hq, lens = 4 * hkv, [33, 700, 1500]
    log(f"decode tok: append-written D={d} P={page} Hkv={hkv}")
    g = torch.Generator().manual_seed(d + page)
    cols = -(-max(lens) // page)
    n_pages = len(lens) * cols + 2
    bt = torch.randperm(n_pages, generator=g)[: len(lens) * cols].view(len(lens), cols).to(torch.int32)
    cache = tuple(t.to(device) for t in (torch.zeros(n_pages, page, hkv, d // 2, dtype=torch.uint8),
                                         torch.zeros(n_pages, page, hkv, d // 2, dtype=torch.uint8),
                                         torch.zeros(n_pages, page, hkv, d // 32, dtype=torch.float16),
                                         torch.zeros(n_pages, page, hkv, d // 32, dtype=torch.float16)))
    cos, sin = workloads.make_rope_cache(max(lens), d)
    gcos, gsin = to(device, cos, sin)
    pos = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens])
    seq = torch.cat([torch.full((n,), b, dtype=torch.int64) for b, n in enumerate(lens)])
    slots = (bt[seq, (pos // page).long()] * page + pos % page).to(torch.int32)
    key = torch.randn(len(pos), hkv, d, generator=g).to(torch.float16)
    val = torch.randn(len(pos), hkv, d, generator=g).to(torch.float16)
    fused_rope_int4_paged_append(*to(device, key, val, pos, slots), gcos, gsin, *cache, rotary_dim=d,
                                 group_size=32, page_size=page)
    torch.cuda.synchronize(device)
    q = torch.randn(len(lens), hq, d, generator=g).to(torch.float16)
    sl = torch.tensor(lens, dtype=torch.int32)
    cpu = tuple(t.cpu() for t in cache)
    for tps in (0, 256):
        _, e32, e16 = _check(device, q, cpu, bt, sl, page, f"append-written D={d} P={page} split={tps}",
                             tokens_per_split=tps)
        log(f"decode tok: append-written D={d} P={page} split={tps}: fp32 {e32:.2e} fp16 {e16:.2e}")


def test_token_pages_positional_handle_and_graph_replay(device):
    # The sync-free positional handle (it plans for the widest batch the
    # block table admits: split-KV here) at head_dim 192 and 8-token pages,
    # then captured in a HIP graph: every replay, with eager work in
    # between, equals the eager launch bit for bit.
    q, cache, bt, sl = _case(16, 2, 192, 8, [500, 1500, 64], 9)
    gq, gbt, gsl = to(device, q, bt, sl)
    gcache = to(device, *cache)
    plan = int4_decode_plan(3, 16, 2, 192, 8, bt.shape[1])
    assert plan[1] > 1 and plan[2] == 8 | DECODE_TOKEN_PAGES, plan
    eager = torch.empty(q.shape, dtype=torch.float32, device=device)
    _int4_paged_decode_attention(gq, *gcache, gbt, gsl, eager, 192, 8)
    torch.cuda.synchronize(device)
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=8, out_dtype=torch.float32)
    assert_attention_close(eager, want, "positional handle D=192 P=8")
    out = torch.empty_like(eager)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        _int4_paged_decode_attention(gq, *gcache, gbt, gsl, out, 192, 8)  # warm-up on the side stream
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _int4_paged_decode_attention(gq, *gcache, gbt, gsl, out, 192, 8)
    for i in range(4):
        out.fill_(float("nan"))
        torch.randn(1000, device=device).sum()  # eager work between replays
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(out, eager), f"replay {i} differs from the eager launch"


def test_token_pages_at_the_benchmark_shape(device):
    # The reference benchmark's B=1 decode shape (Hq=32, Hkv=8, D=128,
    # L=4096) over 16-token pages, on the token-page mode asked for and on
    # the general kernel: the two agree within the attention bound.
    q, cache, bt, sl = _case(32, 8, 128, 16, [4096], 11)
    out, _, _ = _check(device, q, cache, bt, sl, 16, "tok at B=1", waves_per_block=DECODE_TOKEN_PAGES)
    ref, _, _ = _check(device, q, cache, bt, sl, 16, "general at B=1", waves_per_block=4)
    assert_attention_close(out, ref, "tok against the general kernel")


@pytest.mark.parametrize("hq,hkv,d,page", [
    (8, 1, 96, 3),      # odd scale rows (per-token shifts), an odd pool: the any-shape kernel
    (8, 1, 96, 4),      # odd scale rows, an even pool: the token-page mode
    (16, 2, 256, 5),    # head_dim 256: 16-byte scale loads
    (8, 2, 64, 7),      # head_dim 64: 4-byte scale loads
    (8, 2, 128, 1),     # one token a page
    (6, 3, 160, 9),     # odd scale rows, odd pool
])
def test_token_pages_read_the_pool_to_its_last_byte(device, hq, hkv, d, page):
    # Every page of the pool in use and every sequence filling its table
    # row, the pool's last page among them: the loads of the last slot's last
    # kv head end at the tensors' last byte (checked against the eager
    # attention, with and without split-KV).
    lens = [25 * page, 40 * page - 1, 33 * page]
    cols = 40
    g = torch.Generator().manual_seed(d + page + hkv)
    n_pages = len(lens) * cols
    pool = []
    for _ in range(2):
        x = (torch.randn(n_pages, page, hkv, d, generator=g) * 1.5).to(torch.float16)
        codes, scales = quantize_int4_groupwise(x, 32)
        pool.append((pack_int4(codes), scales))
    (kd, ks), (vd, vs) = pool
    perm = torch.randperm(n_pages, generator=g)
    perm = torch.cat([perm[perm != n_pages - 1], torch.tensor([n_pages - 1])])  # the last page last
    bt = perm.view(len(lens), cols).flip(0).contiguous().to(torch.int32)   # ... in sequence 0's row
    q = torch.randn(len(lens), hq, d, generator=g).to(torch.float16)
    sl = torch.tensor(lens, dtype=torch.int32)
    sl[0] = cols * page  # the row's last token lies on the pool's last page
    kw = {"waves_per_block": DECODE_TOKEN_PAGES} if page % 16 == 0 else {}
    for tps in (0, 128):
        _, e32, e16 = _check(device, q, (kd, vd, ks, vs), bt, sl, page,
                             f"pool end Hkv={hkv} D={d} P={page} split={tps}", tokens_per_split=tps, **kw)
        log(f"decode tok: pool end Hkv={hkv} D={d} P={page} split={tps}: fp32 {e32:.2e} fp16 {e16:.2e}")
