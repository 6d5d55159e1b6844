"""Non-finite values inside a sequence's valid range, on every decode kernel.

The eager attention (torch_eager_attention.py:154-239 of the reference)
dequantises code * scale in fp32, so a NaN scale, or an infinite one times a
zero code or summed with mixed signs, makes the logits of every query head of
that kv head NaN; the softmax then turns those heads' whole output rows into
NaN.  A non-finite V scale makes the dims of its 32-dim group non-finite in
every query head of the kv head (NaN, or +-Inf where p > 0 meets a nonzero
code).  A NaN query element makes its head's row NaN.  The kernels must give
the same non-finite positions, NaN wherever the eager result is NaN, and the
finite values within the attention tolerance.  (Where the eager result is
+-Inf -- an infinite V scale with nonzero codes -- the kernels, which remove
the codes' +8 offset by a second sum, give NaN: both are non-finite.)

Each case is run on the plan's own choice, on each INT4 kernel forced (the
streaming kernel at its shapes (4 and 8 query heads per kv head), the MQA
kernel at its shape, the page kernel,
the general kernel and its VALU tile, the kernel of head_dim 96 to 224 and
its token-page mode, the any-shape kernel), with one chunk a sequence and with
split-KV, and on a cache the package's own append wrote from an infinite key
and value.  The FP16-cache decode gets the same check with NaN / Inf cache
values."""
import pytest
import torch

from helpers import ATOL, log, to
from iris_kernel import workloads
from iris_kernel.fused_attention import (DECODE_ANY_KERNEL, DECODE_PAGE_KERNEL, DECODE_TOKEN_PAGES, DECODE_VALU_TILE,
                                         fused_fp16_paged_decode_attention, fused_int4_paged_decode_attention)
from iris_kernel.fused_kv import fused_rope_int4_paged_append
from oracle.torch_eager_attention import (torch_eager_fp16_paged_decode_attention,
                                          torch_eager_int4_paged_decode_attention)
from oracle.torch_eager_kv import pack_int4, quantize_int4_groupwise

pytestmark = pytest.mark.gpu

LENS = [1000, 1500, 2048, 777]
MAX_PAGES = 128  # 2048 tokens a row

# (name, Hq, Hkv, D, waves_per_block): the kernels behind each shape.
KERNELS = [
    ("gqa-auto", 32, 8, 128, 0),
    ("gqa-stream", 32, 8, 128, 16),
    ("gqa-pages", 32, 8, 128, 16 | DECODE_PAGE_KERNEL),
    ("gqa-general", 32, 8, 128, 4),
    ("gqa-valu", 32, 8, 128, 4 | DECODE_VALU_TILE),
    ("gqa8-stream", 64, 8, 128, 16),
    ("gqa8-pages", 64, 8, 128, 16 | DECODE_PAGE_KERNEL),
    ("gqa8-general", 64, 8, 128, 4),
    ("mqa-auto", 16, 1, 64, 0),
    ("mqa-mqa", 16, 1, 64, 16),
    ("mqa-pages", 16, 1, 64, 16 | DECODE_PAGE_KERNEL),
    ("mqa-general", 16, 1, 64, 4),
    ("mqa-valu", 16, 1, 64, 4 | DECODE_VALU_TILE),
    ("gqa-any", 32, 8, 128, DECODE_ANY_KERNEL),
    ("mqa-any", 16, 1, 64, DECODE_ANY_KERNEL),
    ("d96-hd", 8, 2, 96, 0),
    ("d224-hd", 12, 3, 224, 0),
    ("d96-any", 8, 2, 96, DECODE_ANY_KERNEL),
    ("gqa-tok", 32, 8, 128, DECODE_TOKEN_PAGES),
    ("d96-tok", 8, 2, 96, DECODE_TOKEN_PAGES),
    ("d96-tok-odd", 8, 1, 96, DECODE_TOKEN_PAGES),
]

# (name, what is poisoned): sequence b, token t < L_b, kv head, scale group.
CASES = {
    "nan_k": [("k", 0, 500, 1, 2, float("nan"))],
    "inf_k": [("k", 1, 1499, 0, 0, float("inf"))],
    "neg_inf_k": [("k", 2, 3, 3, 1, float("-inf"))],
    "nan_v": [("v", 2, 2047, 2, 3, float("nan"))],
    "inf_v": [("v", 0, 0, 0, 1, float("inf")), ("v", 3, 700, 1, 0, float("-inf"))],
    "nan_q": [("q", 1, None, 5, 17, float("nan"))],
    "mixed": [("k", 3, 776, 2, 0, float("nan")), ("v", 1, 64, 0, 3, float("inf")),
              ("q", 0, None, 0, 3, float("nan"))],
}


def _pool(hkv, d, seed):
    g = torch.Generator().manual_seed(seed)
    n_pages = len(LENS) * MAX_PAGES + 3
    out = []
    for _ in range(2):
        x = (torch.randn(n_pages, 16, hkv, d, generator=g) * 1.5).to(torch.float16)
        codes, scales = quantize_int4_groupwise(x, 32)
        out.append((pack_int4(codes), scales))
    (kd, ks), (vd, vs) = out
    bt = torch.randperm(n_pages, generator=g)[: len(LENS) * MAX_PAGES].view(len(LENS), MAX_PAGES).to(torch.int32)
    return kd, vd, ks, vs, bt


def _poison(case, hq, hkv, d, q, ks, vs, bt):
    q, ks, vs = q.clone(), ks.clone(), vs.clone()
    for what, b, t, h, gidx, val in CASES[case]:
        h = h % (hq if what == "q" else hkv)
        gidx = gidx % (d if what == "q" else d // 32)
        if what == "q":
            q[b, h, gidx] = val
        else:
            page, off = int(bt[b, t // 16]), t % 16
            (ks if what == "k" else vs)[page, off, h, gidx] = val
    return q, ks, vs


def _compare(got, want, what):
    """Same non-finite positions, NaN wherever the eager result is NaN, finite
    values within ATOL."""
    got, want = got.cpu().double(), want.cpu().double()
    bad_got, bad_want = ~torch.isfinite(got), ~torch.isfinite(want)
    assert bad_want.any(), f"{what}: the case poisons nothing in the eager result"
    assert torch.equal(bad_got, bad_want), (
        f"{what}: non-finite at {int(bad_got.sum())} positions, eager at {int(bad_want.sum())}; "
        f"{int((bad_got != bad_want).sum())} differ")
    nan_want = torch.isnan(want)
    assert torch.isnan(got)[nan_want].all(), f"{what}: finite or infinite where the eager result is NaN"
    ok = ~bad_want
    err = (got[ok] - want[ok]).abs().max().item()
    assert err <= ATOL, f"{what}: max-abs err {err:.3e} on the finite positions"
    return int(bad_want.sum()), err


@pytest.mark.parametrize("tps", [0, 256])
@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("name,hq,hkv,d,waves", KERNELS, ids=[k[0] for k in KERNELS])
def test_nonfinite_in_range_matches_eager(device, name, hq, hkv, d, waves, case, tps):
    log(f"nonfinite: {name} case={case} tokens_per_split={tps}")
    kd, vd, ks, vs, bt = _pool(hkv, d, 11 + hq + d)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(len(LENS), hq, d, generator=g).to(torch.float16)
    sl = torch.tensor(LENS, dtype=torch.int32)
    q, ks, vs = _poison(case, hq, hkv, d, q, ks, vs, bt)
    want = torch_eager_int4_paged_decode_attention(q, kd, vd, ks, vs, bt, sl, out_dtype=torch.float32)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(*to(device, q, kd, vd, ks, vs, bt, sl), out, tokens_per_split=tps,
                                      waves_per_block=waves)
    torch.cuda.synchronize(device)
    n_bad, err = _compare(out, want, f"{name} {case} split={tps}")
    # fp16 output: the same positions, rounded finite values
    out16 = torch.empty(q.shape, dtype=torch.float16, device=device)
    fused_int4_paged_decode_attention(*to(device, q, kd, vd, ks, vs, bt, sl), out16, tokens_per_split=tps,
                                      waves_per_block=waves)
    torch.cuda.synchronize(device)
    assert torch.equal(~torch.isfinite(out16.cpu()), ~torch.isfinite(want)), f"{name} {case}: fp16 positions"
    log(f"nonfinite: {name} {case} split={tps}: {n_bad} non-finite positions match, max-abs err {err:.2e}")


@pytest.mark.parametrize("name,hq,hkv,d,waves", KERNELS, ids=[k[0] for k in KERNELS])
def test_append_written_infinite_rows(device, name, hq, hkv, d, waves):
    # The package's append writes an infinite scale and all-zero codes for
    # a group whose amax is infinite (and a NaN scale for a NaN); the eager
    # dequantisation gives 0 * Inf = NaN there.  Rows appended at tokens
    # inside the sequences: an Inf key element (kv head 0), a -Inf value
    # element (kv head hkv - 1) and a NaN key element (another sequence).
    log(f"nonfinite: append-written rows, {name}")
    kd, vd, ks, vs, bt = _pool(hkv, d, 3 + hq)
    g = torch.Generator().manual_seed(6)
    toks = [(0, 10), (2, 1999), (3, 300)]
    key = torch.randn(len(toks), hkv, d, generator=g).to(torch.float16)
    val = torch.randn(len(toks), hkv, d, generator=g).to(torch.float16)
    key[0, 0, 5] = float("inf")
    val[1, hkv - 1, d - 1] = float("-inf")
    key[2, hkv - 1, 40] = float("nan")
    pos = torch.tensor([t for _, t in toks], dtype=torch.int32)
    slots = torch.tensor([int(bt[b, t // 16]) * 16 + t % 16 for b, t in toks], dtype=torch.int32)
    cos, sin = workloads.make_rope_cache(4096, d)
    cache = to(device, kd, vd, ks, vs)
    fused_rope_int4_paged_append(*to(device, key, val, pos, slots, cos, sin), *cache, rotary_dim=d,
                                 group_size=32, page_size=16)
    torch.cuda.synchronize(device)
    kd2, vd2, ks2, vs2 = (t.cpu() for t in cache)
    assert torch.isinf(ks2).any() and torch.isinf(vs2).any() and torch.isnan(ks2).any()
    q = torch.randn(len(LENS), hq, d, generator=g).to(torch.float16)
    sl = torch.tensor(LENS, dtype=torch.int32)
    want = torch_eager_int4_paged_decode_attention(q, kd2, vd2, ks2, vs2, bt, sl, out_dtype=torch.float32)
    for tps in (0, 256):
        out = torch.empty(q.shape, dtype=torch.float32, device=device)
        fused_int4_paged_decode_attention(*to(device, q), *cache, *to(device, bt, sl), out, tokens_per_split=tps,
                                          waves_per_block=waves)
        torch.cuda.synchronize(device)
        n_bad, err = _compare(out, want, f"{name} append-written split={tps}")
        log(f"nonfinite: {name} append-written split={tps}: {n_bad} positions, max-abs err {err:.2e}")


@pytest.mark.parametrize("tps", [0, 256])
@pytest.mark.parametrize("case", ["nan_k", "inf_k", "neg_inf_k", "nan_v", "inf_v", "nan_q"])
def test_fp16_cache_nonfinite_in_range_matches_eager(device, case, tps):
    # The FP16-cache decode over cache values that are NaN or +-Inf (the
    # eager result: an infinite key gives a +-Inf logit, +Inf making its
    # heads NaN and -Inf dropping the token; an infinite value makes its dim
    # non-finite).
    log(f"nonfinite: fp16 cache {case} split={tps}")
    hq, hkv, d = 32, 8, 128
    g = torch.Generator().manual_seed(21)
    n_pages = len(LENS) * MAX_PAGES + 3
    kc = torch.randn(n_pages, 16, hkv, d, generator=g).to(torch.float16)
    vc = torch.randn(n_pages, 16, hkv, d, generator=g).to(torch.float16)
    bt = torch.randperm(n_pages, generator=g)[: len(LENS) * MAX_PAGES].view(len(LENS), MAX_PAGES).to(torch.int32)
    q = torch.randn(len(LENS), hq, d, generator=g).to(torch.float16)
    for what, b, t, h, gidx, val in CASES[case]:
        if what == "q":
            q[b, h % hq, gidx % d] = val
        else:
            page, off = int(bt[b, t // 16]), t % 16
            (kc if what == "k" else vc)[page, off, h % hkv, (32 * gidx + 7) % d] = val
    sl = torch.tensor(LENS, dtype=torch.int32)
    want = torch_eager_fp16_paged_decode_attention(q, kc, vc, bt, sl, out_dtype=torch.float32)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_fp16_paged_decode_attention(*to(device, q, kc, vc, bt, sl), out, tokens_per_split=tps)
    torch.cuda.synchronize(device)
    if not (~torch.isfinite(want)).any():
        # a -Inf logit only drops its token: the result stays finite
        err = (out.cpu().double() - want.double()).abs().max().item()
        assert torch.isfinite(out.cpu()).all() and err <= ATOL, f"fp16 {case}: max-abs err {err:.3e}"
        log(f"nonfinite: fp16 cache {case} split={tps}: finite, max-abs err {err:.2e}")
        return
    n_bad, err = _compare(out, want, f"fp16 {case} split={tps}")
    log(f"nonfinite: fp16 cache {case} split={tps}: {n_bad} positions, max-abs err {err:.2e}")
