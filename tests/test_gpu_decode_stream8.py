"""The streaming decode kernel at 8 query heads per kv head (head_dim 128, 8
kv heads: configuration 5's shape, Llama-3-70B-like GQA) against the
checker's eager attention (fp32 values within helpers.ATOL; fp16 outputs
within one ulp more), on caches quantised as the append writes them.

The kernel runs 16-wave chunk plans of this shape (the plan's choice for
long batches of similar lengths, or any 16-wave request): chunks of up to 64
tiles, the split-KV partials merged in groups of 8 chunks and then across the
groups.  The cases cover one chunk a sequence, one group, several groups,
partial tiles and pages, one-token sequences, pages of 16 << k tokens, both
output types, NaN-poisoned slots past each length, and bit-identical repeats
on one workspace.  Reference: the eager path
(torch_eager_attention.py:154-239); the fused path's shape limits
(fused_attention.py:390-403) allow this shape."""
import pytest
import torch

from helpers import assert_attention_close, log, to
from iris_kernel.fused_attention import DECODE_PAGE_KERNEL, decode_plan, fused_int4_paged_decode_attention
from oracle.torch_eager_attention import torch_eager_int4_paged_decode_attention
from oracle.torch_eager_kv import pack_int4, quantize_int4_groupwise

pytestmark = pytest.mark.gpu

HQ, HKV, D = 64, 8, 128


def _case(page, lens, seed, spare=2):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    max_pages = max(-(-n // page) for n in lens) + 1
    num_pages = B * max_pages + spare
    pool = []
    for _ in range(2):
        x = (torch.randn(num_pages, page, HKV, D, generator=g) * 1.5).to(torch.float16)
        codes, scales = quantize_int4_groupwise(x, 32)
        pool.append((pack_int4(codes), scales))
    (kd, ks), (vd, vs) = pool
    bt = torch.randperm(num_pages, generator=g)[: B * max_pages].view(B, max_pages).to(torch.int32)
    q = torch.randn(B, HQ, D, generator=g).to(torch.float16)
    return q, [kd, vd, ks, vs], bt, torch.tensor(lens, dtype=torch.int32), g


def _launch(device, q, cache, bt, sl, page, tps, out_dtype=torch.float32, waves=16, out=None):
    qg, btg, slg = to(device, q, bt, sl)
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype, device=device)
    fused_int4_paged_decode_attention(qg, *to(device, *cache), btg, slg, out, page_size=page, tokens_per_split=tps,
                                      waves_per_block=waves)
    torch.cuda.synchronize(device)
    return out.cpu()


@pytest.mark.parametrize("page,lens,tps", [
    (16, [4096, 4096, 4096, 4096], 0),        # equal lengths, the plan's split
    (16, [300, 1000], 2048),                  # one chunk a sequence
    (16, [1, 17, 33, 511, 4097], 512),        # 16-tile chunks: up to 9 a sequence, two groups
    (16, [3000, 70, 9000], 1024),             # up to 9 chunks of 32 tiles
    (16, [20000, 5], 512),                    # 40 chunks: five groups
    (16, [65, 2047, 2049], 96),               # chunks of 3 tiles (odd stage counts)
    (32, [40, 1000, 3000], 0),                # 32-token pages
    (64, [130, 5000], 1024),                  # 64-token pages
])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_stream_gqa8_matches_eager(device, page, lens, tps, out_dtype):
    log(f"decode stream g=8: P={page} lens={lens} split={tps} out={out_dtype}")
    q, cache, bt, sl, _ = _case(page, lens, 7 * page + len(lens) + tps)
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=page, out_dtype=torch.float32)
    plan = decode_plan(len(lens), HQ, HKV, D, bt.shape[1] * (page // 16), sum(lens), max(lens), tps, 16)
    assert plan[0] > 0 and plan[1] <= 64 and plan[2] == 16, plan  # a chunk plan the streaming kernel runs
    got = _launch(device, q, cache, bt, sl, page, tps, out_dtype)
    e = assert_attention_close(got, want if out_dtype == torch.float32 else want.to(torch.float16),
                               f"stream g=8 P={page} lens={lens} split={tps}")
    log(f"decode stream g=8: plan {plan} max-abs err {e:.2e}")


def test_stream_gqa8_against_page_kernel(device):
    # The same chunk plan on the page kernel (DECODE_PAGE_KERNEL): another
    # implementation of the same contract, so the two agree within the
    # tolerance and differ in their roundings (two different code paths ran).
    q, cache, bt, sl, _ = _case(16, [1500, 4000, 333], 99)
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=16, out_dtype=torch.float32)
    stream = _launch(device, q, cache, bt, sl, 16, 512)
    pages = _launch(device, q, cache, bt, sl, 16, 512, waves=16 | DECODE_PAGE_KERNEL)
    assert_attention_close(stream, want, "stream g=8")
    assert_attention_close(pages, want, "page kernel g=8")
    assert not torch.equal(stream, pages)


def test_stream_gqa8_nan_tail_and_repeat(device):
    # Slots past each sequence's length hold NaN scales and random codes: the
    # output does not change; a second launch on the same workspace (the
    # arrival counters back at zero) gives the identical result.
    lens = [4100, 30, 777, 2500]
    q, cache, bt, sl, g = _case(16, lens, 4242)
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, sl, page_size=16, out_dtype=torch.float32)
    qg, btg, slg = to(device, q, bt, sl)
    plan = decode_plan(len(lens), HQ, HKV, D, bt.shape[1], sum(lens), max(lens), 256, 16)
    assert plan[1] > 8, plan  # two merge levels
    ws = torch.zeros(plan[3], dtype=torch.uint8, device=device)

    def launch(c):
        out = torch.empty(q.shape, dtype=torch.float32, device=device)
        fused_int4_paged_decode_attention(qg, *to(device, *c), btg, slg, out, tokens_per_split=256,
                                          waves_per_block=16, workspace=ws)
        torch.cuda.synchronize(device)
        return out.cpu()

    clean = launch(cache)
    assert_attention_close(clean, want, "stream g=8 clean")
    assert torch.equal(launch(cache), clean)
    kd, vd, ks, vs = (t.clone() for t in cache)
    for b, n in enumerate(lens):
        last = int(bt[b, (n - 1) // 16])
        tail = slice(n % 16 if n % 16 else 16, 16)
        ks[last, tail] = float("nan")
        vs[last, tail] = float("nan")
        kd[last, tail] = torch.randint(0, 256, kd[last, tail].shape, dtype=torch.uint8, generator=g)
        vd[last, tail] = torch.randint(0, 256, vd[last, tail].shape, dtype=torch.uint8, generator=g)
    poisoned = launch((kd, vd, ks, vs))
    assert torch.isfinite(poisoned).all()
    assert torch.equal(poisoned, clean)
