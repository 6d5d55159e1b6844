"""INT4 decode at head_dim 96, 160, 192 and 224 on the MFMA kernel of
decode_hd.hip: the head dims between the fast kernels' 64, 128 and 256 that
the eager path takes (torch_eager_attention.py:93 of the reference: any
multiple of the 32-dim group) and its fused path refuses
(fused_attention.py:390-403).  Pages of 16 m tokens, any number of kv heads
(odd ones put a kv head's scales on odd halves of their dwords), any number
of query heads per kv head (blocks of 16).  Checked against the checker's
eager attention (fp32 values within helpers.ATOL; fp16 outputs within one
ulp), with one chunk a sequence and with split-KV, and on caches written by
the package's own append."""
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


def _waves(d):
    return 12 if d == 96 else 8


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
    return out, e32, e16


@pytest.mark.parametrize("tps", [0, 128])
@pytest.mark.parametrize("hq,hkv,d,page,lens", [
    (8, 2, 96, 16, [1, 17, 300, 1000]),           # head_dim 96
    (32, 8, 192, 16, [64, 65, 777]),              # head_dim 192
    (16, 2, 160, 32, [100, 2000]),                # head_dim 160, 32-token pages
    (28, 4, 224, 16, [5, 31, 33, 1500]),          # head_dim 224, 7 query heads per kv head
    (8, 2, 96, 48, [47, 48, 49, 2000]),           # 48-token pages
    (40, 2, 96, 48, [77, 1234]),                  # 20 query heads per kv head: two blocks
    (64, 1, 96, 16, [500, 3]),                    # 64 query heads on one kv head: four blocks
    (6, 3, 160, 80, [1, 79, 81, 3000]),           # 3 kv heads (odd scale halves), 80-token pages
    (5, 5, 96, 16, [33, 100, 2]),                 # 5 kv heads, one query head each
    (3, 3, 224, 16, [700, 16, 1]),                # 3 kv heads at head_dim 224
    (16, 1, 192, 256, [1000, 4000]),              # 256-token pages
    (16, 8, 160, 16, [16, 32, 48]),               # whole tiles and a half tile
])
def test_hd_matches_eager(device, hq, hkv, d, page, lens, tps):
    log(f"decode hd: Hq={hq} Hkv={hkv} D={d} P={page} lens={lens} split={tps}")
    q, cache, bt, sl = _case(hq, hkv, d, page, lens, hq * 7 + d + page + tps)
    plan = int4_decode_plan(len(lens), hq, hkv, d, page, bt.shape[1], int(sl.sum()), int(sl.max()), tps)
    assert plan[2] == _waves(d), plan
    _, e32, e16 = _check(device, q, cache, bt, sl, page, f"Hq={hq} Hkv={hkv} D={d} P={page} split={tps}",
                         tokens_per_split=tps)
    log(f"decode hd: max-abs err fp32 {e32:.2e} fp16 {e16:.2e} (plan {plan})")


@pytest.mark.parametrize("d", [96, 160, 192, 224])
def test_hd_agrees_with_the_any_kernel(device, d):
    # The two kernels that serve these head dims, on one case with many
    # chunks: within the same bound of each other as of the eager result.
    q, cache, bt, sl = _case(12, 3, d, 16, [4000, 129, 2500], d)
    out, _, _ = _check(device, q, cache, bt, sl, 16, f"hd D={d}", tokens_per_split=256)
    ref, _, _ = _check(device, q, cache, bt, sl, 16, f"any D={d}", tokens_per_split=256,
                       waves_per_block=DECODE_ANY_KERNEL)
    e = assert_attention_close(out, ref, f"hd against any D={d}")
    log(f"decode hd: D={d} against the any kernel {e:.2e}")


@pytest.mark.parametrize("d,page,hkv", [(96, 16, 4), (160, 16, 3), (224, 48, 1), (192, 32, 2)])
def test_hd_reads_what_the_append_writes(device, d, page, hkv):
    # A cache the package's own append wrote, read back by the decode: the
    # two ends of the path at the same shapes.
    hq, lens = 4 * hkv, [33, 700, 1500]
    log(f"decode hd: append-written D={d} P={page} Hkv={hkv}")
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
        log(f"decode hd: append-written D={d} P={page} split={tps}: fp32 {e32:.2e} fp16 {e16:.2e}")


def test_hd_positional_handle_and_graph_replay(device):
    # The sync-free positional handle (it plans for the widest batch the
    # block table admits: split-KV here) at head_dim 160 and 48-token pages,
    # then captured in a HIP graph: every replay, with eager work in
    # between, equals the eager launch bit for bit.
    q, cache, bt, sl = _case(16, 2, 160, 48, [500, 1500, 64], 9)
    gq, gbt, gsl = to(device, q, bt, sl)
    gcache = to(device, *cache)
    plan = int4_decode_plan(3, 16, 2, 160, 48, bt.shape[1])
    assert plan[1] > 1 and plan[2] == 8, plan
    eager = torch.empty(q.shape, dtype=torch.float32, device=device)
    _int4_paged_decode_attention(gq, *gcache, gbt, gsl, eager, 160, 48)
    torch.cuda.synchronize(device)
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=48, out_dtype=torch.float32)
    assert_attention_close(eager, want, "positional handle D=160 P=48")
    out = torch.empty_like(eager)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        _int4_paged_decode_attention(gq, *gcache, gbt, gsl, out, 160, 48)  # warm-up on the side stream
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _int4_paged_decode_attention(gq, *gcache, gbt, gsl, out, 160, 48)
    for i in range(4):
        out.fill_(float("nan"))
        torch.randn(1000, device=device).sum()  # eager work between replays
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(out, eager), f"replay {i} differs from the eager launch"


def test_hd_workspace_shared_with_other_kernels(device):
    # One caller workspace for split calls whose kernel alternates between
    # the head-dim kernel (D=96, 3 kv heads) and the D=128 kernels, and whose
    # batch grows and shrinks: every kernel keeps its counters at the same
    # place per sequence, and the wrapper zeroes them only when the batch
    # grows past the previous call's.
    ws = torch.zeros(32 << 20, dtype=torch.uint8, device=device)
    cases = {d: _case(12, 3, d, 16, [900, 1500, 64, 2000, 777, 1200, 33, 1800], 40 + d) for d in (96, 128)}
    wants = {d: torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=16, out_dtype=torch.float32)
             for d, (q, cache, bt, sl) in cases.items()}
    gpu = {d: (to(device, q, bt, sl), to(device, *cache)) for d, (q, cache, bt, sl) in cases.items()}
    for d, n, waves in ((96, 8, 0), (128, 4, 4), (96, 8, 0), (128, 8, 16), (96, 2, 0), (128, 8, 4), (96, 5, 0)):
        (gq, gbt, gsl), gcache = gpu[d]
        out = torch.empty(n, 12, d, dtype=torch.float32, device=device)
        fused_int4_paged_decode_attention(gq[:n], *gcache, gbt[:n], gsl[:n], out, tokens_per_split=256,
                                          waves_per_block=waves, workspace=ws)
        torch.cuda.synchronize(device)
        assert_attention_close(out, wants[d][:n], f"D={d} batch {n} waves {waves}")



@pytest.mark.parametrize("hq,hkv,d,page", [(8, 1, 96, 16), (6, 3, 160, 48), (8, 2, 224, 32), (5, 5, 192, 16)])
def test_hd_reads_the_pool_to_its_last_byte(device, hq, hkv, d, page):
    # Every page of the pool in use, the pool's last page at the end of a
    # full table row: the last kv head's code and scale loads of the pool's
    # last token end at the tensors' last byte.
    cols = 24
    g = torch.Generator().manual_seed(d + page + hkv)
    n_pages = 3 * cols
    pool = []
    for _ in range(2):
        x = (torch.randn(n_pages, page, hkv, d, generator=g) * 1.5).to(torch.float16)
        codes, scales = quantize_int4_groupwise(x, 32)
        pool.append((pack_int4(codes), scales))
    (kd, ks), (vd, vs) = pool
    perm = torch.randperm(n_pages, generator=g)
    perm = torch.cat([perm[perm != n_pages - 1], torch.tensor([n_pages - 1])])
    bt = perm.view(3, cols).flip(0).contiguous().to(torch.int32)  # the last page at the end of row 0
    q = torch.randn(3, hq, d, generator=g).to(torch.float16)
    sl = torch.tensor([cols * page, 17 * page - 3, 5 * page], dtype=torch.int32)
    for tps in (0, 128):
        _check(device, q, (kd, vd, ks, vs), bt, sl, page, f"pool end Hkv={hkv} D={d} P={page} split={tps}",
               tokens_per_split=tps)
