"""INT4 decode on the any-shape kernel: head dims that are multiples of 32
(32 to 512; 96, 160, 192 and 224 have an MFMA kernel of their own, and
the token-page mode of that kernel takes every page size at head_dim 64 to
256 by default, so the kernel is asked for here), page sizes that are not
multiples of 16 (one token a page, 8, 24, 40), more than 16 query heads per kv head on such
shapes -- everything the eager path takes (torch_eager_attention.py:72, :93
of the reference) and its fused path refuses (fused_attention.py:390-403).
Checked against the checker's eager attention (fp32 values within
helpers.ATOL; fp16 outputs within one ulp), with one chunk a sequence and
with split-KV, on caches written by the package's own append; plus the
any-shape kernel forced at the fast kernels' shapes, where it must agree
with them."""
import pytest
import torch

from helpers import assert_attention_close, log, to
from iris_kernel import workloads
from iris_kernel.fused_attention import (DECODE_ANY_KERNEL, _int4_paged_decode_attention,
                                         fused_int4_paged_decode_attention, int4_decode_plan)
from iris_kernel.fused_kv import fused_rope_int4_paged_append
from oracle.torch_eager_attention import torch_eager_int4_paged_decode_attention
from oracle.torch_eager_kv import pack_int4, quantize_int4_groupwise

pytestmark = pytest.mark.gpu


def _case(hq, hkv, d, page, lens, seed, spare=3):
    """A paged INT4 pool of random fp16 K/V quantised as the append writes
    it, a shuffled block table wide enough for the longest sequence, and a
    query."""
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
    return e32, e16


@pytest.mark.parametrize("tps", [0, 128])
@pytest.mark.parametrize("hq,hkv,d,page,lens", [
    (8, 2, 96, 16, [1, 17, 300, 1000]),          # head_dim 96
    (32, 8, 192, 16, [64, 65, 777]),              # head_dim 192
    (8, 1, 512, 16, [5, 400, 1300]),              # head_dim 512
    (4, 4, 32, 16, [31, 32, 33, 900]),            # head_dim 32 (one group)
    (16, 2, 160, 32, [100, 2000]),                # odd groups, 32-token pages
    (8, 2, 128, 1, [1, 2, 63, 64, 65, 500]),      # one token a page
    (32, 8, 128, 8, [7, 8, 9, 1111]),             # 8-token pages
    (8, 2, 96, 48, [47, 48, 49, 2000]),           # 48-token pages
    (16, 1, 64, 24, [300, 3000]),                 # MQA at 24-token pages
    (8, 2, 128, 40, [39, 40, 41, 999]),           # 40-token pages
    (40, 2, 96, 48, [77, 1234]),                  # 20 query heads per kv head: two blocks
    (64, 2, 320, 1, [3, 260]),                    # 32 per kv head, head_dim 320, one token a page
])
def test_any_shape_matches_eager(device, hq, hkv, d, page, lens, tps):
    log(f"decode any: Hq={hq} Hkv={hkv} D={d} P={page} lens={lens} split={tps}")
    q, cache, bt, sl = _case(hq, hkv, d, page, lens, hq * 7 + d + page + tps)
    plan = int4_decode_plan(len(lens), hq, hkv, d, page, bt.shape[1], int(sl.sum()), int(sl.max()), tps,
                            DECODE_ANY_KERNEL)
    assert plan[2] & DECODE_ANY_KERNEL, plan
    e32, e16 = _check(device, q, cache, bt, sl, page, f"Hq={hq} Hkv={hkv} D={d} P={page} split={tps}",
                      tokens_per_split=tps, waves_per_block=DECODE_ANY_KERNEL)
    log(f"decode any: max-abs err fp32 {e32:.2e} fp16 {e16:.2e} (plan {plan})")


@pytest.mark.parametrize("d,page", [(96, 16), (192, 48), (512, 1), (32, 8)])
def test_any_shape_reads_what_the_append_writes(device, d, page):
    # A cache the package's own append wrote (head_dim a multiple of 32,
    # any page size), read back by the decode: the two ends of the path at
    # the same shapes.
    hq, hkv, lens = 16, 4, [33, 700, 1500]
    log(f"decode any: append-written D={d} P={page}")
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
        e32, e16 = _check(device, q, cpu, bt, sl, page, f"append-written D={d} P={page} split={tps}",
                          tokens_per_split=tps, waves_per_block=DECODE_ANY_KERNEL)
        log(f"decode any: append-written D={d} P={page} split={tps}: fp32 {e32:.2e} fp16 {e16:.2e}")


@pytest.mark.parametrize("cfg", [1, 3, 4])
def test_any_kernel_forced_at_fast_shapes(device, cfg):
    # The any-shape kernel asked for at the fast kernels' shapes (configs 1,
    # 3, 4 of the benchmark; page size 16): the same contract.
    from helpers import eager_fp32, fill_cpu

    case = workloads.decode_case(cfg)
    log(f"decode any: forced at config {cfg}")
    cpu = fill_cpu(case)
    want = eager_fp32(case, cpu)
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(q, *to(device, *cpu), bt, sl, out, waves_per_block=DECODE_ANY_KERNEL)
    torch.cuda.synchronize(device)
    e = assert_attention_close(out, want, f"any kernel at config {cfg}")
    log(f"decode any: config {cfg} max-abs err {e:.2e}")


def test_positional_handle_at_any_shape(device):
    # The sync-free positional handle plans for the widest batch the block
    # table admits, at a 24-token page and head_dim 288 (the token-page mode
    # takes head dims up to 256).
    q, cache, bt, sl = _case(8, 2, 288, 24, [40, 900], 5)
    assert int4_decode_plan(2, 8, 2, 288, 24, bt.shape[1])[2] & DECODE_ANY_KERNEL
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=24, out_dtype=torch.float32)
    gq, gbt, gsl = to(device, q, bt, sl)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    _int4_paged_decode_attention(gq, *to(device, *cache), gbt, gsl, out, 288, 24)
    torch.cuda.synchronize(device)
    assert_attention_close(out, want, "positional handle D=288 P=24")


def test_hip_graph_replay_at_any_shape(device):
    # The sync-free positional handle at head_dim 320 on one kv head and
    # 8-token pages (split-KV: it plans for the widest batch the table
    # admits), captured in a HIP graph: every replay, with eager work in
    # between, equals the eager launch bit for bit.
    q, cache, bt, sl = _case(16, 1, 320, 8, [500, 1500, 64], 9)
    gq, gbt, gsl = to(device, q, bt, sl)
    gcache = to(device, *cache)
    plan = int4_decode_plan(3, 16, 1, 320, 8, bt.shape[1])
    assert plan[1] > 1 and plan[2] & DECODE_ANY_KERNEL, plan
    eager = torch.empty(q.shape, dtype=torch.float32, device=device)
    _int4_paged_decode_attention(gq, *gcache, gbt, gsl, eager, 320, 8)
    torch.cuda.synchronize(device)
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=8, out_dtype=torch.float32)
    assert_attention_close(eager, want, "graph case eager")
    out = torch.empty_like(eager)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        _int4_paged_decode_attention(gq, *gcache, gbt, gsl, out, 320, 8)  # warm-up on the side stream
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _int4_paged_decode_attention(gq, *gcache, gbt, gsl, out, 320, 8)
    for i in range(4):
        out.fill_(float("nan"))
        torch.randn(1000, device=device).sum()  # eager work between replays
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(out, eager), f"replay {i} differs from the eager launch"
