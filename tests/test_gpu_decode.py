"""INT4 paged decode attention on the GPU against the checker (a restatement
of the reference's torch_eager_int4_paged_decode_attention), on every
benchmark configuration at full size, plus the reference's own scenario,
split-KV invariance, NaN-poisoned tails, GQA ratios, validation errors and
HIP-graph replay.  Tolerance: see helpers.ATOL.

Two kernels sit behind the API: the page-streaming kernel (selected by a
16-wave plan) and the general one (1-4 waves); `KERNELS` runs a test on the
plan's own choice and on each kernel forced.  A shape the page kernel has no
layout for gets the general kernel from a 16-wave request too."""
import math

import pytest
import torch

from helpers import assert_attention_close, eager_fp32, fill_cpu, fill_gpu, log, to
from iris_kernel import workloads
from iris_kernel.fused_attention import (DECODE_PAGE_KERNEL, DECODE_VALU_TILE, _int4_paged_decode_attention,
                                         decode_plan, fused_int4_paged_decode_attention)
from oracle import c_oracle
from oracle.torch_eager_attention import torch_eager_int4_paged_decode_attention

pytestmark = pytest.mark.gpu

_CACHE = {}

# waves_per_block values: 0 = the plan's choice, 16 = page kernel, 4 = general.
KERNELS = {"auto": 0, "pages": 16, "general": 4}


def prepared(cfg, device):
    """(case, cpu cache, gpu cache) for a configuration, built once."""
    if cfg not in _CACHE:
        case = workloads.decode_case(cfg)
        log(f"decode: preparing config {cfg} (B={case.config.batch}, max L={int(case.seq_lens.max())})")
        if cfg == 5:
            gpu = fill_gpu(case, device)
            cpu = tuple(t.cpu() for t in gpu)
        else:
            cpu = fill_cpu(case)
            gpu = to(device, *cpu)
        _CACHE[cfg] = (case, cpu, gpu)
    return _CACHE[cfg]


def run(case, gpu_cache, device, out_dtype=torch.float16, **kw):
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    out = torch.empty(q.shape, dtype=out_dtype, device=device)
    fused_int4_paged_decode_attention(q, *gpu_cache, bt, sl, out, **kw)
    torch.cuda.synchronize(device)
    return out.cpu()


_WANT = {}


@pytest.mark.parametrize("kernel", list(KERNELS))
@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_config_decode_matches_eager(device, cfg, kernel):
    case, cpu, gpu = prepared(cfg, device)
    if cfg not in _WANT:
        log(f"decode: config {cfg} checker")
        _WANT[cfg] = eager_fp32(case, cpu)
    want32 = _WANT[cfg]
    w = KERNELS[kernel]
    got32 = run(case, gpu, device, torch.float32, waves_per_block=w)
    e32 = assert_attention_close(got32, want32, f"cfg{cfg} {kernel} fp32")
    got16 = run(case, gpu, device, waves_per_block=w)
    e16 = assert_attention_close(got16, want32.to(torch.float16), f"cfg{cfg} {kernel} fp16")
    log(f"decode: config {cfg} {kernel} max-abs err fp32 {e32:.2e} fp16 {e16:.2e}")


@pytest.mark.parametrize("cfg", [2, 3])
def test_page_kernel_forced_matches_eager(device, cfg):
    # At the streaming kernel's shape a 16-wave plan runs the streaming
    # kernel (chunk mode at cfg2, balanced mode at cfg3); the
    # DECODE_PAGE_KERNEL bit keeps the page-streaming kernel, which must
    # hold the same contract.
    case, cpu, gpu = prepared(cfg, device)
    if cfg not in _WANT:
        _WANT[cfg] = eager_fp32(case, cpu)
    got = run(case, gpu, device, torch.float32, waves_per_block=16 | DECODE_PAGE_KERNEL)
    e = assert_attention_close(got, _WANT[cfg], f"cfg{cfg} page kernel forced")
    log(f"decode: config {cfg} page kernel forced max-abs err {e:.2e}")


@pytest.mark.parametrize("kernel", list(KERNELS))
def test_config5_long_context_against_float64(device, kernel):
    # L = 131072 per sequence: the float64 C checker (the torch one would
    # materialise 4 GB per sequence for the GQA expansion).
    case, cpu, gpu = prepared(5, device)
    if 5 not in _WANT:
        log("decode: config 5 float64 checker")
        _WANT[5] = c_oracle.decode_f64(case.query, *cpu, case.block_table, case.seq_lens)
    want = _WANT[5]
    w = KERNELS[kernel]
    got32 = run(case, gpu, device, torch.float32, waves_per_block=w)
    e32 = assert_attention_close(got32, want, f"cfg5 {kernel} fp32")
    got16 = run(case, gpu, device, waves_per_block=w)
    e16 = assert_attention_close(got16, want.to(torch.float16), f"cfg5 {kernel} fp16")
    log(f"decode: config 5 {kernel} max-abs err fp32 {e32:.2e} fp16 {e16:.2e}")


def test_reference_attention_scenario(device):
    # test_attention.py:16-196: B=2, Hq=8, Hkv=2, D=128, L=[23, 31] (partial
    # pages and a partial 32-token tile), randperm page table with 3 spares.
    torch.manual_seed(3407)
    B, Hq, Hkv, D, P = 2, 8, 2, 128, 16
    lens = torch.tensor([23, 31], dtype=torch.int32)
    NP = B * 2 + 3
    bt = torch.randperm(NP)[: B * 2].reshape(B, 2).to(torch.int32)
    cos, sin = workloads.make_rope_cache(31, D)
    cache = (torch.zeros(NP, P, Hkv, D // 2, dtype=torch.uint8), torch.zeros(NP, P, Hkv, D // 2, dtype=torch.uint8),
             torch.zeros(NP, P, Hkv, D // 32, dtype=torch.float16), torch.zeros(NP, P, Hkv, D // 32, dtype=torch.float16))
    for b in range(B):
        n = int(lens[b])
        key = torch.randn(n, Hkv, D, dtype=torch.float16)
        value = torch.randn_like(key)
        pos = torch.arange(n, dtype=torch.int32)
        slots = (bt[b, (pos // P).long()] * P + pos % P).to(torch.int32)
        c_oracle.append(key, value, pos, slots, cos, sin, *cache, rotary_dim=D, group_size=32, page_size=16)
    q = torch.randn(B, Hq, D, dtype=torch.float16)
    want = torch_eager_int4_paged_decode_attention(q, *cache, bt, lens, out_dtype=torch.float32)
    out = fused_int4_paged_decode_attention(*to(device, q, *cache, bt, lens))
    torch.cuda.synchronize(device)
    assert_attention_close(out, want.to(torch.float16), "reference scenario")


@pytest.mark.parametrize("waves", [16, 4])
@pytest.mark.parametrize("tokens_per_split", [32, 96, 512, 1024, 0])
def test_split_kv_invariance(device, tokens_per_split, waves):
    # The split count changes only rounding: each split rescales p by its own
    # running max before p * v_scale is rounded to fp16 (at most 2^-11
    # relative per term, independent across terms), so two plans agree to
    # a few 1e-4 on config 1/2 outputs; each plan is separately held to the
    # 2e-3 contract against eager by the config tests.
    # (32 tokens a split: 128 chunks a sequence, so the page kernel merges in
    # two levels.)
    case, cpu, gpu = prepared(2, device)
    base = run(case, gpu, device, torch.float32, tokens_per_split=4096, waves_per_block=4)
    got = run(case, gpu, device, torch.float32, tokens_per_split=tokens_per_split, waves_per_block=waves)
    assert (got - base).abs().max().item() < 5e-4


@pytest.mark.parametrize("tokens_per_split", [256, 1024])
def test_split_kv_invariance_head_dim_64(device, tokens_per_split):
    # Configuration 4 (D=64, 16 query heads per kv head) on the general
    # kernel: at 256 tokens a split a sequence has 32 chunks, four merge
    # batches of 8 (the batch at D=64); at 1024, 8 chunks in one batch.
    # Against the plan with the fewest chunks (4).
    case, cpu, gpu = prepared(4, device)
    base = run(case, gpu, device, torch.float32, tokens_per_split=8192, waves_per_block=4)
    got = run(case, gpu, device, torch.float32, tokens_per_split=tokens_per_split, waves_per_block=4)
    assert (got - base).abs().max().item() < 1e-3


def _ragged_lens(case):
    g = torch.Generator().manual_seed(7 + len(case))
    if case == "log-uniform":
        return (2 ** (7 + 7 * torch.rand(64, generator=g))).round().to(torch.int32)
    if case == "one-long":
        return torch.tensor([16384] + [128] * 63, dtype=torch.int32)
    if case == "many-tiny":
        return torch.randint(1, 41, (1500,), generator=g, dtype=torch.int32)
    return torch.tensor([100000, 7, 100000], dtype=torch.int32)  # "two-huge"


@pytest.mark.parametrize("case", ["log-uniform", "one-long", "many-tiny", "two-huge"])
def test_balanced_split_ragged_batches(device, case):
    # Ragged lengths through the public wrapper (lengths known) put the page
    # kernel in its balanced mode: equal shares of all sequences' tiles, a
    # sequence cut where the shares meet it.  Cases: configuration 3's
    # length law; one 16K sequence among short ones (more than 8 chunks: the
    # second merge level); 1500 sequences of 1-40 tokens (several a share,
    # and a scan longer than one workgroup); two 100K-token sequences around
    # a 7-token one.  Checked against the float64 C checker, twice on one
    # workspace (counters back at zero after a call).
    lens = _ragged_lens(case)
    B, Hq, Hkv, D = lens.numel(), 32, 8, 128
    g = torch.Generator().manual_seed(11)
    pages = [(int(L) + 15) // 16 for L in lens]
    maxp = max(pages)
    NP = sum(pages) + 1
    perm = torch.randperm(NP, generator=g).to(torch.int32)
    bt = torch.full((B, maxp), int(perm[-1]), dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    kd = torch.randint(0, 256, (NP, 16, Hkv, D // 2), dtype=torch.uint8, generator=g)
    vd = torch.randint(0, 256, (NP, 16, Hkv, D // 2), dtype=torch.uint8, generator=g)
    ks = (torch.rand(NP, 16, Hkv, D // 32, generator=g) * 0.3).to(torch.float16)
    vs = (torch.rand(NP, 16, Hkv, D // 32, generator=g) * 0.3).to(torch.float16)
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    plan = decode_plan(B, Hq, Hkv, D, maxp, int(lens.sum()), int(lens.max()), 0, 16)
    assert plan[2] == 16 and plan[0] < 0, plan  # the balanced mode
    want = c_oracle.decode_f64(q, kd, vd, ks, vs, bt, lens)
    args = to(device, q, kd, vd, ks, vs, bt, lens)
    ws = torch.zeros(max(plan[3], 1), dtype=torch.uint8, device=device)
    for i in range(2):
        out = torch.empty(q.shape, dtype=torch.float32, device=device)
        fused_int4_paged_decode_attention(*args, out, waves_per_block=16, workspace=ws)
        torch.cuda.synchronize(device)
        assert_attention_close(out, want, f"{case} call {i}")


@pytest.mark.parametrize("kernel", ["stream", "pages"])
def test_stale_balanced_plan_writes_nan(device, kernel):
    # A balanced plan made for short ragged lengths, launched (through the
    # C ABI's launch path) with lengths whose tiles exceed what its ranges
    # can cover: every output element is NaN, not a silently truncated
    # result, and the workspace stays usable for the next correct call.  At
    # this shape the streaming kernel's balanced mode runs the plan, or the
    # page-streaming kernel with the DECODE_PAGE_KERNEL bit.
    from iris_kernel import fused_attention as fa

    waves = 16 | (DECODE_PAGE_KERNEL if kernel == "pages" else 0)

    case, cpu, gpu = prepared(2, device)
    q, bt, full = to(device, case.query, case.block_table, case.seq_lens)
    B, hq, d = q.shape
    short = torch.full((B,), 40, dtype=torch.int32)
    short[0] = 70
    plan = decode_plan(B, hq, 8, d, bt.shape[1], int(short.sum()), int(short.max()), 0, waves)
    assert plan[0] < 0 and plan[2] == waves, plan
    # the full lengths outgrow it (the streaming kernel counts 3 more units a sequence)
    assert 32 * (4096 // 32) > 64 * plan[1], plan
    ws = torch.zeros(max(plan[3], 1), dtype=torch.uint8, device=device)
    out = torch.empty(B, hq, d, dtype=torch.float32, device=device)
    fa._launch_decode(q, *gpu, bt, short.to(device), out, d ** -0.5, plan, ws)
    torch.cuda.synchronize(device)
    assert_attention_close(out, eager_fp32(case, cpu, seq_lens=short), "planned lengths")
    for dtype in (torch.float32, torch.float16):
        bad = torch.zeros(B, hq, d, dtype=dtype, device=device)
        fa._launch_decode(q, *gpu, bt, full, bad, d ** -0.5, plan, ws)
        torch.cuda.synchronize(device)
        assert torch.isnan(bad.float()).all(), f"{dtype}: a stale plan must poison every output"
    fa._launch_decode(q, *gpu, bt, short.to(device), out, d ** -0.5, plan, ws)
    torch.cuda.synchronize(device)
    assert_attention_close(out, eager_fp32(case, cpu, seq_lens=short), "after the stale call")


def test_workspace_across_batches_and_kernels(device):
    # One workspace for calls whose batch grows and shrinks and whose kernel
    # changes (page kernel, general kernel): the counters sit at a fixed
    # place per sequence, and the wrapper zeroes the counter region only when
    # the batch grows past the previous call's.
    case, cpu, gpu = prepared(2, device)
    if 2 not in _WANT:
        _WANT[2] = eager_fp32(case, cpu)
    want = _WANT[2]
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=device)
    for n, waves in ((32, 16), (4, 16), (32, 4), (8, 4), (32, 16), (1, 16), (32, 4)):
        out = torch.empty(n, q.shape[1], q.shape[2], dtype=torch.float32, device=device)
        fused_int4_paged_decode_attention(q[:n], *gpu, bt[:n], sl[:n], out, waves_per_block=waves,
                                          tokens_per_split=512, workspace=ws)
        torch.cuda.synchronize(device)
        assert_attention_close(out, want[:n], f"batch {n} waves {waves}")


@pytest.mark.parametrize("waves", [1, 2, 3, 4, 16])
def test_waves_per_block_invariance(device, waves):
    case, cpu, gpu = prepared(1, device)
    base = run(case, gpu, device, torch.float32, waves_per_block=4, tokens_per_split=64)
    got = run(case, gpu, device, torch.float32, waves_per_block=waves, tokens_per_split=64)
    assert (got - base).abs().max().item() < 5e-4


@pytest.mark.parametrize("waves", [16, 4])
def test_nan_poisoned_tails_do_not_leak(device, waves):
    # Configuration 3 (ragged, partial last pages, shuffled pool): poison
    # every slot past each sequence's length and the unused pad page with
    # NaN scales and random bytes; results must not change.
    case, cpu, gpu = prepared(3, device)
    clean = run(case, gpu, device, torch.float32, waves_per_block=waves)
    kd, vd, ks, vs = (t.clone() for t in cpu)
    g = torch.Generator().manual_seed(99)
    for b in range(case.config.batch):
        n = int(case.seq_lens[b])
        last = int(case.block_table[b, (n - 1) // 16])
        tail = slice(n % 16 if n % 16 else 16, 16)
        ks[last, tail] = float("nan")
        vs[last, tail] = float("nan")
        kd[last, tail] = torch.randint(0, 256, kd[last, tail].shape, dtype=torch.uint8, generator=g)
        vd[last, tail] = torch.randint(0, 256, vd[last, tail].shape, dtype=torch.uint8, generator=g)
    ks[case.pad_page] = float("nan")
    vs[case.pad_page] = float("inf")
    poisoned = run(case, to(device, kd, vd, ks, vs), device, torch.float32, waves_per_block=waves)
    assert torch.isfinite(poisoned).all()
    assert torch.equal(poisoned, clean)


@pytest.mark.parametrize("waves", [0, 16])
@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (4, 2, 64), (12, 4, 128), (10, 2, 64), (24, 3, 128),
                                      (16, 2, 128), (32, 2, 64), (16, 1, 128), (6, 6, 64), (32, 8, 64),
                                      (4, 1, 128), (16, 4, 64)])
def test_gqa_ratios_and_head_dims(device, hq, hkv, d, waves):
    g = torch.Generator().manual_seed(hq * 100 + hkv + d)
    B, maxp = 3, 9
    NP = B * maxp + 2
    bt = torch.randperm(NP, generator=g)[: B * maxp].view(B, maxp).to(torch.int32)
    lens = torch.tensor([1, 77, 144], dtype=torch.int32)
    kd = torch.randint(0, 256, (NP, 16, hkv, d // 2), dtype=torch.uint8, generator=g)
    vd = torch.randint(0, 256, (NP, 16, hkv, d // 2), dtype=torch.uint8, generator=g)
    ks = (torch.rand(NP, 16, hkv, d // 32, generator=g) * 0.5).to(torch.float16)
    vs = (torch.rand(NP, 16, hkv, d // 32, generator=g) * 0.5).to(torch.float16)
    q = torch.randn(B, hq, d, generator=g).to(torch.float16)
    want = torch_eager_int4_paged_decode_attention(q, kd, vd, ks, vs, bt, lens, out_dtype=torch.float32)
    out = torch.empty(B, hq, d, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(*to(device, q, kd, vd, ks, vs, bt, lens), out, waves_per_block=waves)
    torch.cuda.synchronize(device)
    assert_attention_close(out, want, f"hq={hq} hkv={hkv} d={d} waves={waves}")


def test_custom_softmax_scale_and_private_handle(device):
    case, cpu, gpu = prepared(1, device)
    want = torch_eager_int4_paged_decode_attention(case.query, *cpu, case.block_table, case.seq_lens,
                                                   softmax_scale=0.3, out_dtype=torch.float32)
    got = run(case, gpu, device, torch.float32, softmax_scale=0.3)
    assert_attention_close(got, want, "softmax_scale=0.3")
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    _int4_paged_decode_attention(q, *gpu, bt, sl, out, 64, 16, 32, 16, 32, 128, 0.0)
    torch.cuda.synchronize(device)
    assert_attention_close(out, eager_fp32(case, cpu), "private handle")


def test_zero_softmax_scale_and_strided_inputs(device):
    # The reference wrapper hands softmax_scale=0.0 to its kernel, which
    # reads 0.0 as head_dim ** -0.5 (fused_attention.py:50, :523): an
    # explicit 0.0 gives the default result.  Strided inputs (q split out of
    # a fused qkv tensor, a block_table column slice, a strided seq_lens)
    # give the same result as dense ones.
    case, cpu, gpu = prepared(1, device)
    want = eager_fp32(case, cpu)
    got = run(case, gpu, device, torch.float32, softmax_scale=0.0)
    assert_attention_close(got, want, "softmax_scale=0.0")
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    B, hq, d = q.shape
    qkv = torch.empty(B, 3 * hq, d, dtype=q.dtype, device=device)
    qkv[:, :hq] = q
    wide_bt = torch.full((B, bt.shape[1] + 5), -1, dtype=torch.int32, device=device)
    wide_bt[:, :bt.shape[1]] = bt
    sl2 = torch.stack([sl, torch.zeros_like(sl)], dim=1)[:, 0]
    assert not qkv[:, :hq].is_contiguous() and not wide_bt[:, :bt.shape[1]].is_contiguous()
    assert not sl2.is_contiguous()
    out = torch.empty(B, hq, d, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(qkv[:, :hq], *gpu, wide_bt[:, :bt.shape[1]], sl2, out)
    torch.cuda.synchronize(device)
    assert_attention_close(out, want, "strided inputs")


def test_validation_errors(device):
    case, cpu, gpu = prepared(1, device)
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    with pytest.raises(ValueError):
        fused_int4_paged_decode_attention(q, *gpu, bt, torch.zeros_like(sl))
    too_long = sl.clone()
    too_long[0] = bt.shape[1] * 16 + 1
    with pytest.raises(ValueError):
        fused_int4_paged_decode_attention(q, *gpu, bt, too_long)
    bad_bt = bt.clone()
    bad_bt[1, 0] = case.num_pages
    with pytest.raises(IndexError):
        fused_int4_paged_decode_attention(q, *gpu, bad_bt, sl)
    with pytest.raises(TypeError):
        fused_int4_paged_decode_attention(q, *gpu, bt.to(torch.int16), sl)
    with pytest.raises(TypeError):
        fused_int4_paged_decode_attention(q.float(), *gpu, bt, sl)
    # int64 ids and lengths past the int32 range are still invalid, as in the reference
    huge_bt = bt.long()
    huge_bt[1, 0] = 2 ** 32 + 1  # would wrap to page 1 if narrowed naively
    with pytest.raises(IndexError):
        fused_int4_paged_decode_attention(q, *gpu, huge_bt, sl.long())
    huge_sl = sl.long()
    huge_sl[0] = 2 ** 40
    with pytest.raises(ValueError):
        fused_int4_paged_decode_attention(q, *gpu, bt.long(), huge_sl)
    with pytest.raises(NotImplementedError):
        fused_int4_paged_decode_attention(q, *gpu, bt, sl, group_size=64)
    with pytest.raises(ValueError):
        fused_int4_paged_decode_attention(q, *gpu, bt, sl, torch.empty(1, device=device))


@pytest.mark.parametrize("cfg", [1, 3])
def test_int64_metadata_matches_int32(device, cfg):
    # int64 block_table / seq_lens, accepted like the eager path
    # (torch_eager_attention.py:130-133): the same result as int32.
    case, cpu, gpu = prepared(cfg, device)
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    want = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(q, *gpu, bt, sl, want)
    for bt_x, sl_x in ((bt.long(), sl.long()), (bt.long(), sl), (bt, sl.long())):
        got = torch.empty_like(want)
        fused_int4_paged_decode_attention(q, *gpu, bt_x, sl_x, got)
        torch.cuda.synchronize(device)
        assert torch.equal(got, want)


def test_hip_graph_replay(device):
    # The sync-free private handle captured in a HIP graph: every replay,
    # with eager work in between, must equal the eager launch.
    case, cpu, gpu = prepared(2, device)
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    eager = torch.empty(q.shape, dtype=torch.float16, device=device)
    _int4_paged_decode_attention(q, *gpu, bt, sl, eager, 128, 16)
    torch.cuda.synchronize(device)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        _int4_paged_decode_attention(q, *gpu, bt, sl, out, 128, 16)  # warm-up on the side stream
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _int4_paged_decode_attention(q, *gpu, bt, sl, out, 128, 16)
    for i in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(out, eager), f"replay {i}"


# ------------------------------------------------------------------ wider scope
def _quantized_pool(num_pages, page_size, hkv, d, gen):
    """A cache pool of random fp16 K/V quantised as the append writes it."""
    from oracle.torch_eager_kv import pack_int4, quantize_int4_groupwise
    out = []
    for _ in range(2):
        x = (torch.randn(num_pages, page_size, hkv, d, generator=gen) * 1.5).to(torch.float16)
        codes, scales = quantize_int4_groupwise(x, 32)
        out.append((pack_int4(codes), scales))
    (kd, ks), (vd, vs) = out
    return kd, vd, ks, vs


@pytest.mark.parametrize("kernel", list(KERNELS))
@pytest.mark.parametrize("hq,hkv,d,page,lens,tps", [
    (16, 4, 256, 16, [1, 300, 1000], 0),        # head_dim 256
    (16, 4, 256, 16, [700, 1200], 128),
    (32, 1, 128, 16, [50, 900, 2000], 0),       # 32 query heads per kv head
    (48, 2, 64, 16, [333, 1500], 256),          # 24 per kv head: a full and a half block
    (20, 1, 128, 16, [77, 555], 0),
    (32, 8, 128, 32, [40, 1000, 3000], 0),      # 32-token pages
    (32, 8, 128, 32, [2100, 3000], 256),
    (8, 2, 128, 64, [1, 100, 700], 0),          # 64-token pages
    (16, 4, 64, 128, [130, 5000], 512),         # 128-token pages
    (32, 8, 128, 256, [4000, 17], 0),           # 256-token pages
])
def test_wider_scope_matches_eager(device, kernel, hq, hkv, d, page, lens, tps):
    # Shapes the reference's fused decode rejects (fused_attention.py:390-403)
    # and its eager path computes: held to the same tolerance.
    log(f"decode scope: Hq={hq} Hkv={hkv} D={d} P={page} lens={lens} split={tps} kernel={kernel}")
    g = torch.Generator().manual_seed(hq * 7 + d + page + len(lens))
    B = len(lens)
    max_pages = max(-(-n // page) for n in lens) + 1
    num_pages = B * max_pages + 2
    kd, vd, ks, vs = _quantized_pool(num_pages, page, hkv, d, g)
    bt = torch.randperm(num_pages, generator=g)[: B * max_pages].view(B, max_pages).to(torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.float16)
    want = torch_eager_int4_paged_decode_attention(q, kd, vd, ks, vs, bt, sl, page_size=page,
                                                   out_dtype=torch.float32)
    qg, btg, slg = to(device, q, bt, sl)
    cache = to(device, kd, vd, ks, vs)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(qg, *cache, btg, slg, out, page_size=page, tokens_per_split=tps,
                                      waves_per_block=KERNELS[kernel])
    torch.cuda.synchronize(device)
    assert_attention_close(out, want, f"Hq={hq} Hkv={hkv} D={d} P={page}")


# ------------------------------------------------------------------ MQA streaming kernel
# One kv head, head_dim 64, at most 16 query heads: 16-wave plans run the MQA
# streaming kernel (decode_mqa.hip).  Ragged lengths (partial tiles and
# pages, a one-token sequence, steps with fewer tiles than waves), splits of
# 1 to many chunks, fewer query heads than MFMA columns, pages of 16 << k
# tokens, fp32 and fp16 outputs.
# Pages of 16 m tokens with m not a power of two (48, 80, 144, 240): the
# fast kernels read a page as m consecutive 16-token pages, looked up with
# a division instead of a shift; each kernel choice, with and without
# split-KV, against the eager attention.
@pytest.mark.parametrize("kernel", ["auto", "wave16", "pages", "general"])
@pytest.mark.parametrize("hq,hkv,d,page,lens,tps", [
    (32, 8, 128, 48, [47, 48, 49, 1500, 3001], 0),
    (32, 8, 128, 80, [100, 2000], 256),
    (16, 1, 64, 144, [143, 145, 5000], 512),     # one kv head: the MQA kernel at 16 waves
    (64, 8, 128, 240, [239, 4000], 0),           # 8 query heads per kv head
    (16, 4, 128, 48, [900, 10, 2500], 1024),
])
def test_page_sizes_multiple_of_16_match_eager(device, kernel, hq, hkv, d, page, lens, tps):
    from iris_kernel.fused_attention import int4_decode_plan
    waves = {"auto": 0, "wave16": 16, "pages": 16 | DECODE_PAGE_KERNEL, "general": 4}[kernel]
    log(f"decode: P={page} Hq={hq} Hkv={hkv} D={d} lens={lens} split={tps} kernel={kernel}")
    g = torch.Generator().manual_seed(page * 3 + hq + len(lens) + tps)
    B = len(lens)
    cols = max(-(-n // page) for n in lens) + 1
    num_pages = B * cols + 2
    kd, vd, ks, vs = _quantized_pool(num_pages, page, hkv, d, g)
    bt = torch.randperm(num_pages, generator=g)[: B * cols].view(B, cols).to(torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.float16)
    plan = int4_decode_plan(B, hq, hkv, d, page, cols, sum(lens), max(lens), tps, waves)
    assert not plan[2] & 0x400, plan  # a fast kernel, not the any-shape one
    want = torch_eager_int4_paged_decode_attention(q, kd, vd, ks, vs, bt, sl, page_size=page,
                                                   out_dtype=torch.float32)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(*to(device, q, kd, vd, ks, vs, bt, sl), out, page_size=page,
                                      tokens_per_split=tps, waves_per_block=waves)
    torch.cuda.synchronize(device)
    e = assert_attention_close(out.cpu(), want, f"P={page} Hq={hq} Hkv={hkv} D={d} {kernel} plan={plan}")
    log(f"decode: P={page} {kernel} plan {plan} max-abs err {e:.2e}")


@pytest.mark.parametrize("hq,page,lens,tps", [
    (16, 16, [8192, 8192, 8192], 0),          # configuration 4's shape, plan's split
    (16, 16, [1, 17, 33, 511, 4097], 0),
    (16, 16, [1, 17, 33, 511, 4097], 512),    # 16-tile chunks: many per sequence
    (16, 16, [3000, 70, 9000], 1536),         # chunks of 48 tiles (three steps)
    (8, 16, [600, 2500], 0),                  # half the columns
    (3, 16, [129, 1000, 31], 512),
    (1, 16, [2000], 0),
    (16, 32, [40, 1000, 3000], 0),            # 32-token pages
    (12, 128, [130, 5000], 1024),             # 128-token pages
])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_mqa_kernel_matches_eager(device, hq, page, lens, tps, out_dtype):
    log(f"decode mqa: Hq={hq} P={page} lens={lens} split={tps} out={out_dtype}")
    g = torch.Generator().manual_seed(hq * 11 + page + len(lens) + tps)
    B = len(lens)
    max_pages = max(-(-n // page) for n in lens) + 1
    num_pages = B * max_pages + 2
    kd, vd, ks, vs = _quantized_pool(num_pages, page, 1, 64, g)
    bt = torch.randperm(num_pages, generator=g)[: B * max_pages].view(B, max_pages).to(torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(B, hq, 64, generator=g).to(torch.float16)
    want = torch_eager_int4_paged_decode_attention(q, kd, vd, ks, vs, bt, sl, page_size=page,
                                                   out_dtype=torch.float32)
    plan = decode_plan(B, hq, 1, 64, max_pages * (page // 16), sum(lens), max(lens), tps, 16)
    assert plan[2] == 16 and plan[0] % 16 == 0, plan  # the MQA kernel's plan: whole steps of 16 tiles
    qg, btg, slg = to(device, q, bt, sl)
    cache = to(device, kd, vd, ks, vs)
    out = torch.empty(q.shape, dtype=out_dtype, device=device)
    fused_int4_paged_decode_attention(qg, *cache, btg, slg, out, page_size=page, tokens_per_split=tps,
                                      waves_per_block=16)
    torch.cuda.synchronize(device)
    assert_attention_close(out.cpu(), want if out_dtype == torch.float32 else want.to(torch.float16),
                           f"mqa Hq={hq} P={page} lens={lens}")


def test_mqa_kernel_nan_tail_and_repeat(device):
    # Slots past each sequence's length hold NaN scales and random codes: the
    # output must not change; a second launch on the same workspace (the
    # arrival counters back at zero) gives the identical result.
    g = torch.Generator().manual_seed(4242)
    lens = [4100, 30, 777]
    B, hq, page = len(lens), 16, 16
    max_pages = max(-(-n // page) for n in lens) + 1
    num_pages = B * max_pages + 2
    kd, vd, ks, vs = _quantized_pool(num_pages, page, 1, 64, g)
    bt = torch.randperm(num_pages, generator=g)[: B * max_pages].view(B, max_pages).to(torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(B, hq, 64, generator=g).to(torch.float16)
    want = torch_eager_int4_paged_decode_attention(q, kd, vd, ks, vs, bt, sl, page_size=page,
                                                   out_dtype=torch.float32)
    qg, btg, slg = to(device, q, bt, sl)

    def launch(cache):
        out = torch.empty(q.shape, dtype=torch.float32, device=device)
        fused_int4_paged_decode_attention(qg, *to(device, *cache), btg, slg, out, tokens_per_split=512,
                                          waves_per_block=16)
        torch.cuda.synchronize(device)
        return out.cpu()

    clean = launch((kd, vd, ks, vs))
    assert_attention_close(clean, want, "mqa clean")
    assert torch.equal(launch((kd, vd, ks, vs)), clean)
    kd, vd, ks, vs = (t.clone() for t in (kd, vd, ks, vs))
    for b, n in enumerate(lens):
        last = int(bt[b, (n - 1) // page])
        tail = slice(n % page if n % page else page, page)
        ks[last, tail] = float("nan")
        vs[last, tail] = float("nan")
        kd[last, tail] = torch.randint(0, 256, kd[last, tail].shape, dtype=torch.uint8, generator=g)
        vd[last, tail] = torch.randint(0, 256, vd[last, tail].shape, dtype=torch.uint8, generator=g)
    poisoned = launch((kd, vd, ks, vs))
    assert torch.isfinite(poisoned).all()
    assert torch.equal(poisoned, clean)


# ------------------------------------------------------------------ VALU tile
# DECODE_VALU_TILE: the general kernel with v_dot2c chains (DPP row
# broadcasts) in place of its MFMAs -- the alternative the MFMA tile is
# measured against -- held to the same contract on the layouts it covers
# (g = 4 at D = 128 with four kv heads a wave, g = 16 at D = 64).
@pytest.mark.parametrize("cfg", [2, 3, 4])
def test_valu_tile_matches_eager(device, cfg):
    case, cpu, gpu = prepared(cfg, device)
    if cfg not in _WANT:
        log(f"decode: config {cfg} checker")
        _WANT[cfg] = eager_fp32(case, cpu)
    want32 = _WANT[cfg]
    got32 = run(case, gpu, device, torch.float32, waves_per_block=4 | DECODE_VALU_TILE)
    e32 = assert_attention_close(got32, want32, f"cfg{cfg} valu fp32")
    got16 = run(case, gpu, device, waves_per_block=4 | DECODE_VALU_TILE)
    e16 = assert_attention_close(got16, want32.to(torch.float16), f"cfg{cfg} valu fp16")
    log(f"decode: config {cfg} valu max-abs err fp32 {e32:.2e} fp16 {e16:.2e}")


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 1, 64)])
@pytest.mark.parametrize("tps", [0, 96, 1024])
def test_valu_tile_ragged_and_split(device, hq, hkv, d, tps):
    # Lengths with partial pages and partial 32-token tiles (1, 17, 33), a
    # full table row and one token short of it; one chunk, 3-tile chunks
    # (43 a sequence) and 32-tile chunks.
    lens = [1, 17, 33, 1000, 4095, 4096]
    log(f"decode valu: Hq={hq} Hkv={hkv} D={d} lens={lens} split={tps}")
    g = torch.Generator().manual_seed(hq + d + tps)
    B, max_pages = len(lens), 257
    num_pages = B * max_pages + 2
    kd, vd, ks, vs = _quantized_pool(num_pages, 16, hkv, d, g)
    bt = torch.randperm(num_pages, generator=g)[: B * max_pages].view(B, max_pages).to(torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.float16)
    want = torch_eager_int4_paged_decode_attention(q, kd, vd, ks, vs, bt, sl, out_dtype=torch.float32)
    qg, btg, slg = to(device, q, bt, sl)
    cache = to(device, kd, vd, ks, vs)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    fused_int4_paged_decode_attention(qg, *cache, btg, slg, out, tokens_per_split=tps, waves_per_block=4 | DECODE_VALU_TILE)
    torch.cuda.synchronize(device)
    assert_attention_close(out, want, f"valu Hq={hq} Hkv={hkv} D={d} split={tps}")


def test_valu_tile_nan_poisoned_tails(device):
    # As test_nan_poisoned_tails_do_not_leak, on the VALU tile.
    case, cpu, gpu = prepared(3, device)
    clean = run(case, gpu, device, torch.float32, waves_per_block=4 | DECODE_VALU_TILE)
    kd, vd, ks, vs = (t.clone() for t in cpu)
    g = torch.Generator().manual_seed(98)
    for b in range(case.config.batch):
        n = int(case.seq_lens[b])
        last = int(case.block_table[b, (n - 1) // 16])
        tail = slice(n % 16 if n % 16 else 16, 16)
        ks[last, tail] = float("nan")
        vs[last, tail] = float("nan")
        kd[last, tail] = torch.randint(0, 256, kd[last, tail].shape, dtype=torch.uint8, generator=g)
        vd[last, tail] = torch.randint(0, 256, vd[last, tail].shape, dtype=torch.uint8, generator=g)
    ks[case.pad_page] = float("nan")
    vs[case.pad_page] = float("inf")
    poisoned = run(case, to(device, kd, vd, ks, vs), device, torch.float32, waves_per_block=4 | DECODE_VALU_TILE)
    assert torch.isfinite(poisoned).all()
    assert torch.equal(poisoned, clean)


def test_recycled_workspace_block_is_zeroed(device):
    # A caller's workspace tensor placed by the caching allocator where an
    # earlier workspace was, after other data (0xFF bytes) passed through
    # that block: the wrapper has never seen the new tensor, so it zero-fills
    # its counter region, every merge runs, and the result is the checker's.
    case, cpu, gpu = prepared(2, device)
    if 2 not in _WANT:
        _WANT[2] = eager_fp32(case, cpu)
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    B, hq, d = q.shape
    lens = case.seq_lens.tolist()
    nbytes = decode_plan(B, hq, 8, d, bt.shape[1], sum(lens), max(lens))[3]
    assert nbytes > 0
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    first = torch.empty(nbytes, dtype=torch.uint8, device=device)
    fused_int4_paged_decode_attention(q, *gpu, bt, sl, out, workspace=first)
    torch.cuda.synchronize(device)
    assert_attention_close(out, _WANT[2], "first workspace")
    where = first.data_ptr()
    del first
    junk = torch.empty(nbytes, dtype=torch.uint8, device=device)
    junk.fill_(0xFF)
    torch.cuda.synchronize(device)
    del junk
    second = torch.empty(nbytes, dtype=torch.uint8, device=device)
    if second.data_ptr() != where:  # (another block: the same test on the junk bytes themselves)
        second.fill_(0xFF)
    out.fill_(0.0)
    fused_int4_paged_decode_attention(q, *gpu, bt, sl, out, workspace=second)
    torch.cuda.synchronize(device)
    log(f"decode: recycled workspace block, same address: {second.data_ptr() == where}")
    assert_attention_close(out, _WANT[2], "recycled workspace")
