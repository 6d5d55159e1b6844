"""iris_int4_paged_decode_attention_noalloc (split-KV workspace inside the
library, nothing allocated) against iris_int4_paged_decode_attention with a
caller workspace, through the C ABI: bit-identical outputs on two calls in a
row, the second with a smaller input, and a plan too large for the library's
array rejected with IRIS_ERR_WORKSPACE."""
import ctypes

import pytest
import torch

from helpers import log
from iris_kernel import _lib
from iris_kernel import fused_attention as fa
from iris_kernel.fused_attention import decode_plan

pytestmark = pytest.mark.gpu

IRIS_ERR_WORKSPACE = 3
SCRATCH_BYTES = 8 << 20


def random_cache(num_pages, hkv, d, gen):
    """A random INT4 cache: codes in [-7, 7] packed low nibble first, scales in [0.02, 0.5)."""
    codes = torch.randint(-7, 8, (2, num_pages, 16, hkv, d), generator=gen, dtype=torch.int16)
    nib = codes & 0xF
    packed = (nib[..., 0::2] | (nib[..., 1::2] << 4)).to(torch.uint8)
    scales = (torch.rand((2, num_pages, 16, hkv, d // 32), generator=gen) * 0.48 + 0.02).to(torch.float16)
    return packed[0], packed[1], scales[0], scales[1]


def make_case(batch, hq, hkv, d, max_pages, max_len, gen):
    num_pages = batch * max_pages + 3
    cache = random_cache(num_pages, hkv, d, gen)
    perm = torch.randperm(num_pages, generator=gen)[: batch * max_pages]
    bt = perm.view(batch, max_pages).to(torch.int32)
    sl = torch.randint(max_len // 3, max_len + 1, (batch,), generator=gen, dtype=torch.int32)
    sl[0] = max_len
    q = torch.randn((batch, hq, d), generator=gen).to(torch.float16)
    return q, cache, bt, sl


def noalloc_call(q, cache, bt, sl, out, scale, plan):
    chunk_tiles, max_chunks, nw, _ = plan
    batch, hq, d = q.shape
    num_pages, page_size, hkv, _ = cache[0].shape
    return _lib.lib().iris_int4_paged_decode_attention_noalloc(
        q.data_ptr(), cache[0].data_ptr(), cache[1].data_ptr(), cache[2].data_ptr(), cache[3].data_ptr(),
        bt.data_ptr(), sl.data_ptr(), out.data_ptr(), 0, batch, hq, hkv, d, page_size, num_pages, bt.shape[1],
        ctypes.c_float(scale), chunk_tiles, max_chunks, nw, _lib.raw_stream(q.device))


def one_call(device, batch, max_pages, max_len, tokens_per_split, seed, hq=32, hkv=8, d=128, waves=0):
    gen = torch.Generator().manual_seed(seed)
    q, cache, bt, sl = make_case(batch, hq, hkv, d, max_pages, max_len, gen)
    q, bt, sl = (t.to(device) for t in (q, bt, sl))
    cache = tuple(t.to(device) for t in cache)
    plan = decode_plan(batch, hq, hkv, d, max_pages, int(sl.sum()), int(sl.max()), tokens_per_split, waves)
    assert plan[1] > 1 and 0 < plan[3] <= SCRATCH_BYTES, plan
    if waves & 0xFF:
        assert plan[2] == waves, plan
    elif waves:  # a selection bit alone: the plan names the wave count
        assert plan[2] & ~0xFF == waves, plan
    log(f"no-alloc: batch={batch} hq={hq} hkv={hkv} d={d} max_len={max_len} plan={plan}")
    scale = d ** -0.5
    want = torch.empty(q.shape, dtype=torch.float16, device=device)
    fa._launch_decode(q, *cache, bt, sl, want, scale, plan)
    got = torch.full(q.shape, float("nan"), dtype=torch.float16, device=device)
    status = noalloc_call(q, cache, bt, sl, got, scale, plan)
    assert status == 0, status
    torch.cuda.synchronize(device)
    assert torch.isfinite(want).all()
    assert torch.equal(got.cpu(), want.cpu())


def test_noalloc_matches_workspace_entry_two_calls(device):
    one_call(device, batch=12, max_pages=96, max_len=1536, tokens_per_split=256, seed=11)
    one_call(device, batch=5, max_pages=48, max_len=700, tokens_per_split=128, seed=12)


def test_noalloc_streaming_kernels_two_calls(device):
    """16-wave plans: the streaming kernel (Hkv 8, D 128, ragged lengths) and
    the MQA kernel (one kv head, D 64), each larger call then smaller."""
    one_call(device, batch=8, max_pages=256, max_len=4096, tokens_per_split=0, seed=21, waves=16)
    one_call(device, batch=3, max_pages=128, max_len=2048, tokens_per_split=0, seed=22, waves=16)
    one_call(device, batch=16, max_pages=512, max_len=8192, tokens_per_split=0, seed=23, hq=16, hkv=1, d=64,
             waves=16)
    one_call(device, batch=6, max_pages=256, max_len=4096, tokens_per_split=0, seed=24, hq=16, hkv=1, d=64,
             waves=16)


def test_noalloc_head_dim_and_any_shape_kernels_two_calls(device):
    """The head_dim 96-224 kernel (the plan's choice at 96 and 224) and the
    any-shape kernel (asked for, at 160), each larger call then smaller."""
    one_call(device, batch=8, max_pages=128, max_len=2048, tokens_per_split=256, seed=31, hq=16, hkv=4, d=96)
    one_call(device, batch=3, max_pages=64, max_len=1000, tokens_per_split=256, seed=32, hq=16, hkv=4, d=96)
    one_call(device, batch=6, max_pages=96, max_len=1536, tokens_per_split=256, seed=33, hq=12, hkv=3, d=224)
    one_call(device, batch=2, max_pages=32, max_len=500, tokens_per_split=128, seed=34, hq=12, hkv=3, d=224)
    one_call(device, batch=5, max_pages=64, max_len=1024, tokens_per_split=256, seed=35, hq=8, hkv=2, d=160,
             waves=0x400)
    one_call(device, batch=2, max_pages=32, max_len=400, tokens_per_split=128, seed=36, hq=8, hkv=2, d=160,
             waves=0x400)


def test_noalloc_token_pages_two_calls(device):
    """The head-dim kernel's token-page mode (asked for at head_dim 128 and
    64, 16-token pages), each larger call then smaller."""
    one_call(device, batch=8, max_pages=128, max_len=2048, tokens_per_split=256, seed=41, hq=32, hkv=8, d=128,
             waves=0x800)
    one_call(device, batch=3, max_pages=64, max_len=900, tokens_per_split=128, seed=42, hq=32, hkv=8, d=128,
             waves=0x800)
    one_call(device, batch=6, max_pages=96, max_len=1536, tokens_per_split=256, seed=43, hq=16, hkv=1, d=64,
             waves=0x800)
    one_call(device, batch=2, max_pages=64, max_len=900, tokens_per_split=128, seed=44, hq=16, hkv=1, d=64,
             waves=0x800)


def test_noalloc_rejects_plan_beyond_scratch(device):
    batch, hq, hkv, d, max_pages = 64, 32, 8, 128, 256
    plan = decode_plan(batch, hq, hkv, d, max_pages, batch * max_pages * 16, max_pages * 16, 64, 0)
    assert plan[3] > SCRATCH_BYTES, plan
    q = torch.zeros((batch, hq, d), dtype=torch.float16, device=device)
    cache = tuple(torch.zeros(s, dtype=t, device=device)
                  for s, t in (((1, 16, hkv, d // 2), torch.uint8), ((1, 16, hkv, d // 2), torch.uint8),
                               ((1, 16, hkv, d // 32), torch.float16), ((1, 16, hkv, d // 32), torch.float16)))
    bt = torch.zeros((batch, max_pages), dtype=torch.int32, device=device)
    sl = torch.full((batch,), max_pages * 16, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    assert noalloc_call(q, cache, bt, sl, out, d ** -0.5, plan) == IRIS_ERR_WORKSPACE
    torch.cuda.synchronize(device)
