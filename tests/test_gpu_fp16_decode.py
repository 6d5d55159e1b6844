"""FP16 paged decode attention (the reference's matched FP16 baseline) on the
GPU, through the C ABI, against the checker's restatement of
torch_eager_fp16_paged_decode_attention: benchmark configurations 1-4 at
full size, the reference's attention scenario with its INT4-vs-FP16 quality
gate (tests/test_attention.py:199-232), split invariance, NaN-poisoned
tails, GQA ratios, validation errors, the positional handle and HIP-graph
replay.  Tolerance: helpers.ATOL (2e-3 max-abs on fp32 outputs; fp16 outputs
max(2e-3, one fp16 ulp of the reference value))."""
import pytest
import torch

from helpers import assert_attention_close, log, to
from iris_kernel import workloads
from iris_kernel.fused_attention import (_fp16_paged_decode_attention, fused_fp16_paged_decode_attention,
                                         fused_int4_paged_decode_attention)
from oracle.torch_eager_attention import torch_eager_int4_paged_decode_attention
from oracle import c_oracle
from oracle.torch_eager_attention import torch_eager_fp16_paged_decode_attention
from oracle.torch_eager_kv import apply_rope

pytestmark = pytest.mark.gpu

_CACHE = {}


def fp16_cache(case, device):
    """fp16 cache [NP, 16, Hkv, D] of a decode case: RoPE(K) and V at every
    prefill slot (what the FP16 append writes), zeros elsewhere."""
    c = case.config
    shape = (case.num_pages, 16, c.num_kv_heads, c.head_dim)
    kc = torch.zeros(shape, dtype=torch.float16, device=device)
    vc = torch.zeros(shape, dtype=torch.float16, device=device)

    def append(k, v, p, s, cos, sin, kc, vc):
        rk = apply_rope(k, cos[p.long()][:, None, :], sin[p.long()][:, None, :], rotary_dim=c.head_dim)
        kc.view(-1, c.num_kv_heads, c.head_dim)[s.long()] = rk
        vc.view(-1, c.num_kv_heads, c.head_dim)[s.long()] = v

    case.fill_cache(append, (kc, vc), device=device)
    torch.cuda.synchronize(device)
    return kc, vc


def prepared(cfg, device):
    if cfg not in _CACHE:
        case = workloads.decode_case(cfg)
        log(f"fp16 decode: preparing config {cfg} (B={case.config.batch}, max L={int(case.seq_lens.max())})")
        gpu = fp16_cache(case, device)
        cpu = tuple(t.cpu() for t in gpu)
        _CACHE[cfg] = (case, cpu, gpu)
    return _CACHE[cfg]


def run(case, gpu_cache, device, out_dtype=torch.float16, **kw):
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    out = torch.empty(q.shape, dtype=out_dtype, device=device)
    fused_fp16_paged_decode_attention(q, *gpu_cache, bt, sl, out, **kw)
    torch.cuda.synchronize(device)
    return out.cpu()


def eager(case, cpu_cache, out_dtype=torch.float32, **kw):
    return torch_eager_fp16_paged_decode_attention(case.query, *cpu_cache, case.block_table, case.seq_lens,
                                                   out_dtype=out_dtype, **kw)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_fp16_config_decode_matches_eager(device, cfg):
    case, cpu, gpu = prepared(cfg, device)
    want32 = eager(case, cpu)
    got32 = run(case, gpu, device, torch.float32)
    e32 = assert_attention_close(got32, want32, f"fp16 cfg{cfg} fp32")
    got16 = run(case, gpu, device)
    e16 = assert_attention_close(got16, want32.to(torch.float16), f"fp16 cfg{cfg} fp16")
    log(f"fp16 decode: config {cfg} max-abs err fp32 {e32:.2e} fp16 {e16:.2e}")


def _reference_case():
    # test_attention.py:16-162: B=2, Hq=8, Hkv=2, D=128, L=[23, 31], randperm
    # page table with 3 spare pages; the INT4 cache from the eager append and
    # the FP16 cache from RoPE(K) and V at the same slots; query rotated at
    # position L - 1.
    torch.manual_seed(3407)
    B, Hq, Hkv, D, P = 2, 8, 2, 128, 16
    lens = torch.tensor([23, 31], dtype=torch.int32)
    NP = B * 2 + 3
    bt = torch.randperm(NP)[: B * 2].reshape(B, 2).to(torch.int32)
    cos, sin = workloads.make_rope_cache(31, D)
    int4 = (torch.zeros(NP, P, Hkv, D // 2, dtype=torch.uint8), torch.zeros(NP, P, Hkv, D // 2, dtype=torch.uint8),
            torch.zeros(NP, P, Hkv, D // 32, dtype=torch.float16), torch.zeros(NP, P, Hkv, D // 32, dtype=torch.float16))
    kc = torch.zeros(NP, P, Hkv, D, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    for b in range(B):
        n = int(lens[b])
        key = torch.randn(n, Hkv, D, dtype=torch.float16)
        value = torch.randn_like(key)
        pos = torch.arange(n, dtype=torch.int32)
        slots = (bt[b, (pos // P).long()] * P + pos % P).to(torch.int32)
        rk = apply_rope(key, cos[pos.long()][:, None, :], sin[pos.long()][:, None, :], rotary_dim=D)
        kc[slots.long() // P, slots.long() % P] = rk
        vc[slots.long() // P, slots.long() % P] = value
        c_oracle.append(key, value, pos, slots, cos, sin, *int4, rotary_dim=D, group_size=32, page_size=16)
    qpos = (lens - 1).long()
    q_raw = torch.randn(B, Hq, D, dtype=torch.float16)
    q = apply_rope(q_raw, cos[qpos][:, None, :], sin[qpos][:, None, :], rotary_dim=D)
    return q, bt, lens, int4, (kc, vc)


def test_fp16_reference_scenario_and_int4_quality_gate(device):
    q, bt, lens, int4, fp16 = _reference_case()
    want = torch_eager_fp16_paged_decode_attention(q, *fp16, bt, lens, out_dtype=torch.float32)
    out16 = fused_fp16_paged_decode_attention(*to(device, q, *fp16, bt, lens))
    out4 = fused_int4_paged_decode_attention(*to(device, q, *int4, bt, lens))
    torch.cuda.synchronize(device)
    assert_attention_close(out16, want.to(torch.float16), "fp16 reference scenario")
    # test_attention.py:203-232 on the two GPU paths: the INT4 cache tracks
    # the FP16 one.
    a, b = out4.float().cpu().flatten(0, 1), out16.float().cpu().flatten(0, 1)
    cosine = torch.nn.functional.cosine_similarity(a, b, dim=-1).mean().item()
    rmse = torch.mean((a - b) ** 2).sqrt().item()
    log(f"fp16 decode: reference scenario INT4 vs FP16 cosine {cosine:.4f} rmse {rmse:.4f}")
    assert cosine > 0.97
    assert rmse < 0.20


@pytest.mark.parametrize("tokens_per_split", [16, 64, 256, 1024, 0])
def test_fp16_split_invariance(device, tokens_per_split):
    # Splits change only rounding (each split's p is rounded to fp16 against
    # its own running max), so plans agree to a few 1e-4 on config 2.
    case, cpu, gpu = prepared(2, device)
    base = run(case, gpu, device, torch.float32, tokens_per_split=1 << 20)
    got = run(case, gpu, device, torch.float32, tokens_per_split=tokens_per_split)
    assert (got - base).abs().max().item() < 5e-4


def test_fp16_nan_poisoned_tails_do_not_leak(device):
    # Configuration 3 (ragged, partial last pages): NaN / inf in every slot
    # past each sequence and in the pad page must not change the result.
    case, cpu, gpu = prepared(3, device)
    clean = run(case, gpu, device, torch.float32)
    kc, vc = (t.clone() for t in cpu)
    for b in range(case.config.batch):
        n = int(case.seq_lens[b])
        last = int(case.block_table[b, (n - 1) // 16])
        tail = slice(n % 16 if n % 16 else 16, 16)
        kc[last, tail] = float("nan")
        vc[last, tail] = float("nan")
    kc[case.pad_page] = float("inf")
    vc[case.pad_page] = float("nan")
    poisoned = run(case, to(device, kc, vc), device, torch.float32)
    assert torch.isfinite(poisoned).all()
    assert torch.equal(poisoned, clean)


@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (4, 2, 64), (12, 4, 128), (10, 2, 64), (24, 3, 128),
                                      (16, 1, 128), (32, 2, 64), (6, 6, 64), (64, 8, 128), (16, 4, 64)])
def test_fp16_gqa_ratios_and_head_dims(device, hq, hkv, d):
    g = torch.Generator().manual_seed(hq * 100 + hkv + d)
    B, maxp = 3, 9
    NP = B * maxp + 2
    bt = torch.randperm(NP, generator=g)[: B * maxp].view(B, maxp).to(torch.int32)
    lens = torch.tensor([1, 77, 144], dtype=torch.int32)
    kc = torch.randn(NP, 16, hkv, d, generator=g).to(torch.float16)
    vc = torch.randn(NP, 16, hkv, d, generator=g).to(torch.float16)
    q = torch.randn(B, hq, d, generator=g).to(torch.float16)
    want = torch_eager_fp16_paged_decode_attention(q, kc, vc, bt, lens, out_dtype=torch.float32)
    for tps in (0, 32):
        out = torch.empty(B, hq, d, dtype=torch.float32, device=device)
        fused_fp16_paged_decode_attention(*to(device, q, kc, vc, bt, lens), out, tokens_per_split=tps)
        torch.cuda.synchronize(device)
        assert_attention_close(out, want, f"fp16 hq={hq} hkv={hkv} d={d} tps={tps}")


# The page-streaming kernel (decode_fp16_stream.hip: head_dim 128 with 4 or 8
# kv heads, head_dim 64 with 8 or 16; the plan's choice there for batches of
# similar lengths and for unknown lengths, so these ragged batches take its
# plan from the block table's width): partial tiles and pages, one-token
# sequences, one to 16 chunks, 4 to 16 query heads per kv head, both output
# types.
@pytest.mark.parametrize("hq,hkv,d,lens,tps", [
    (32, 8, 128, [1, 9, 16, 17, 300, 2049], 0),
    (32, 8, 128, [1, 9, 16, 17, 300, 2049], 128),   # 8-page chunks (16 a sequence at most)
    (16, 4, 128, [5000, 33], 1024),
    (64, 8, 128, [3000, 8], 256),                    # 8 query heads per kv head
    (128, 8, 64, [700, 1500], 0),                    # head_dim 64, 16 per kv head
    (16, 16, 64, [40, 2000, 777], 512),              # 16 kv heads
])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_fp16_page_streaming_kernel_matches_eager(device, hq, hkv, d, lens, tps, out_dtype):
    from iris_kernel.fused_attention import _launch_fp16_decode, fp16_decode_plan
    g = torch.Generator().manual_seed(hq + hkv + d + len(lens) + tps)
    B = len(lens)
    maxp = max(-(-n // 16) for n in lens) + 1
    NP = B * maxp + 2
    bt = torch.randperm(NP, generator=g)[: B * maxp].view(B, maxp).to(torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    kc = torch.randn(NP, 16, hkv, d, generator=g).to(torch.float16)
    vc = torch.randn(NP, 16, hkv, d, generator=g).to(torch.float16)
    q = torch.randn(B, hq, d, generator=g).to(torch.float16)
    # these small batches ask for the kernel (negative tokens_per_split;
    # left to choose, the plan gives batches under 8 sequences or 64 MB the
    # per-kv-head kernel)
    plan = fp16_decode_plan(B, hq, hkv, d, maxp, -1, -1, -(tps or 1024))
    assert -128 <= plan[0] < 0 and plan[1] <= 16, plan  # the page-streaming kernel's plan
    assert fp16_decode_plan(B, hq, hkv, d, maxp, sum(lens), max(lens), tps)[0] > 0  # ragged: the other kernel
    want = torch_eager_fp16_paged_decode_attention(q, kc, vc, bt, sl, out_dtype=torch.float32)
    out = torch.empty(B, hq, d, dtype=out_dtype, device=device)
    _launch_fp16_decode(*to(device, q, kc, vc, bt, sl), out, d ** -0.5, plan)
    torch.cuda.synchronize(device)
    assert_attention_close(out, want if out_dtype == torch.float32 else want.to(torch.float16),
                           f"fp16 stream hq={hq} hkv={hkv} d={d} lens={lens} tps={tps} plan={plan}")


def test_fp16_softmax_scale_and_private_handle(device):
    case, cpu, gpu = prepared(1, device)
    want = eager(case, cpu, softmax_scale=0.3)
    got = run(case, gpu, device, torch.float32, softmax_scale=0.3)
    assert_attention_close(got, want, "fp16 softmax_scale=0.3")
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    out = torch.empty(q.shape, dtype=torch.float32, device=device)
    _fp16_paged_decode_attention(q, *gpu, bt, sl, out, 64, 16, 16, 32, 128, 0.0)
    torch.cuda.synchronize(device)
    assert_attention_close(out, eager(case, cpu), "fp16 private handle")


def test_fp16_validation_errors(device):
    # fused_attention.py:528-566 and :373-434: the same exception types.
    case, cpu, gpu = prepared(1, device)
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    kc, vc = gpu
    with pytest.raises(ValueError):
        fused_fp16_paged_decode_attention(q, kc, vc[:-1], bt, sl)
    with pytest.raises(ValueError):
        fused_fp16_paged_decode_attention(q, kc[..., :32], vc[..., :32], bt, sl)
    with pytest.raises(ValueError):
        fused_fp16_paged_decode_attention(q, kc, vc, bt, torch.zeros_like(sl))
    bad_bt = bt.clone()
    bad_bt[1, 0] = case.num_pages
    with pytest.raises(IndexError):
        fused_fp16_paged_decode_attention(q, kc, vc, bad_bt, sl)
    with pytest.raises(TypeError):
        fused_fp16_paged_decode_attention(q, kc.float(), vc.float(), bt, sl)
    with pytest.raises(TypeError):
        fused_fp16_paged_decode_attention(q, kc, vc, bt.to(torch.int16), sl)
    want = fused_fp16_paged_decode_attention(q, kc, vc, bt, sl)  # int64 metadata: the same result
    assert torch.equal(fused_fp16_paged_decode_attention(q, kc, vc, bt.long(), sl.long()), want)
    with pytest.raises(ValueError):  # the cache's page dimension is checked first
        fused_fp16_paged_decode_attention(q, kc, vc, bt, sl, page_size=32)
    np_, _, hkv, d = kc.shape
    with pytest.raises(NotImplementedError):  # a 32-token page cache: outside the fast path
        fused_fp16_paged_decode_attention(q, kc.view(np_ // 2, 32, hkv, d), vc.view(np_ // 2, 32, hkv, d),
                                          bt, sl, page_size=32)
    with pytest.raises(ValueError):
        fused_fp16_paged_decode_attention(q, kc, vc, bt, sl, torch.empty(1, device=device))


def test_fp16_hip_graph_replay(device):
    case, cpu, gpu = prepared(2, device)
    q, bt, sl = to(device, case.query, case.block_table, case.seq_lens)
    eager_out = torch.empty(q.shape, dtype=torch.float16, device=device)
    _fp16_paged_decode_attention(q, *gpu, bt, sl, eager_out, 128, 16)
    torch.cuda.synchronize(device)
    out = torch.empty_like(eager_out)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        _fp16_paged_decode_attention(q, *gpu, bt, sl, out, 128, 16)
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _fp16_paged_decode_attention(q, *gpu, bt, sl, out, 128, 16)
    for i in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(out, eager_out), f"replay {i}"


def test_split_workspace_shared_by_kernels_and_layouts(device):
    # One stream, one cached workspace, three kernels whose counters and
    # partials sit at different offsets (B=32: the FP16 kernel's counters
    # span bytes the INT4 page kernel fills with partials), interleaved and
    # each with splits; every call must still match its checker.
    g = torch.Generator().manual_seed(77)
    B, Hq, Hkv, D, L = 32, 32, 8, 128, 512
    maxp = L // 16
    NP = B * maxp
    bt = torch.randperm(NP, generator=g).view(B, maxp).to(torch.int32)
    lens = torch.full((B,), L, dtype=torch.int32)
    lens[::3] = 300
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    int4 = (torch.randint(0, 256, (NP, 16, Hkv, D // 2), dtype=torch.uint8, generator=g),
            torch.randint(0, 256, (NP, 16, Hkv, D // 2), dtype=torch.uint8, generator=g),
            (torch.rand(NP, 16, Hkv, D // 32, generator=g) * 0.2).to(torch.float16),
            (torch.rand(NP, 16, Hkv, D // 32, generator=g) * 0.2).to(torch.float16))
    f16 = (torch.randn(NP, 16, Hkv, D, generator=g).to(torch.float16),
           torch.randn(NP, 16, Hkv, D, generator=g).to(torch.float16))
    want4 = torch_eager_int4_paged_decode_attention(q, *int4, bt, lens, out_dtype=torch.float32)
    want16 = torch_eager_fp16_paged_decode_attention(q, *f16, bt, lens, out_dtype=torch.float32)
    qd, btd, ld = to(device, q, bt, lens)
    i4d, f16d = to(device, *int4), to(device, *f16)
    calls = [("int4 pages", lambda o: fused_int4_paged_decode_attention(qd, *i4d, btd, ld, o, waves_per_block=16,
                                                                        tokens_per_split=128), want4),
             ("fp16", lambda o: fused_fp16_paged_decode_attention(qd, *f16d, btd, ld, o, tokens_per_split=128), want16),
             ("int4 general", lambda o: fused_int4_paged_decode_attention(qd, *i4d, btd, ld, o, waves_per_block=4,
                                                                          tokens_per_split=64), want4),
             ("fp16 other split", lambda o: fused_fp16_paged_decode_attention(qd, *f16d, btd, ld, o,
                                                                              tokens_per_split=96), want16)]
    for rnd in range(2):
        for name, fn, want in calls:
            out = torch.empty(B, Hq, D, dtype=torch.float32, device=device)
            fn(out)
            torch.cuda.synchronize(device)
            assert_attention_close(out, want, f"round {rnd} {name}")
