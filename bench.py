#!/usr/bin/env python3
"""Benchmark of the INT4 paged KV-cache hot path on one MI355X.

Metric: INT4 paged decode-attention us + HBM GB/s (% of
peak) at B=32, L=4K; append tokens/s.

Workload (configuration 2, Llama-3-8B-shaped single layer): Hq=32, Hkv=8,
D=128, batch 32, every sequence at context 4096, page size 16, randomly
permuted pages, fp16 N(0,1) synthetic data.  One step = the fused RoPE+INT4
append of 32 new tokens (one per sequence, position 4095) followed by INT4
paged decode attention over the 4096 tokens.

* The cache is replicated (--replicas, default: enough copies to exceed
  600 MB) and steps rotate through the copies, so every decode reads its
  151.6 MB from HBM, not from the 256 MB Infinity Cache.
* ``ms_per_step``: wall clock over exactly K steps bracketed by
  torch.cuda.synchronize() (kernel launches included).
* Op times: HIP events on the launch stream around each op, in a second
  pass where a GPU sleep lets the host queue every step first, so the events
  bracket kernel execution only (``append_us``).
* Decode kernel time: one event pair around K back-to-back decode launches
  on the launch stream (rotating over the replicas, after 5 untimed ones),
  i.e. the average launch duration of the single decode kernel (split-KV
  combine fused in); the median of 3 such passes (all in
  ``decode_us_passes``).  ``value`` = algorithmic decode bytes / that
  duration.
* ``roofline.traffic``: HBM bytes per decode launch measured with rocprofv3
  counters (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), read from
  profiles/decode_cfg2_traffic.json.
* ``fp16_decode``: the same decode over an fp16 cache (the reference's
  matched FP16 baseline), timed the same way; ``int4_speedup`` is its time
  over the INT4 decode's.
* ``cpu_baseline``: the checker's restatements of the reference's PyTorch
  eager decode and append (oracle/), timed on this host's cores on bounded
  samples of the same workloads (decode GB/s as ``value``; the step's
  append and a sample of the configuration-5 bulk append in tokens/s), with
  the host's CPU model.

--gpus N > 1 exits: this path is measured on one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT / "iris-kernel_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
METRIC = "INT4 paged decode-attn µs + HBM GB/s (% of peak) at B=32,4K; append tokens/s"


def decode_bytes(batch, n_q, n_kv, d, lens) -> int:
    """Compulsory bytes of one decode: packed K+V (D bytes per token and kv
    head) + K/V scales (D/8) + q in and o out (fp16) + block-table entries
    read + seq_lens."""
    kv = sum(lens) * n_kv * (d + d // 8)
    return kv + 2 * batch * n_q * d * 2 + 4 * sum((n + 15) // 16 for n in lens) + 4 * batch


def append_bytes(n_tok, n_kv, d, n_pos) -> int:
    """Compulsory bytes of one append: K and V in (fp16), positions and
    slots, packed codes + scales out, one cos and one sin row per distinct
    position."""
    return n_tok * (4 * n_kv * d + 8 + n_kv * (d + d // 8)) + n_pos * 2 * d


def decode_kernel_name(plan, group: int, n_kv: int, d: int, batch: int, max_pages: int) -> str:
    """Name of the decode kernel a plan runs, as rocprofv3 reports it.  16-wave
    plans: the streaming kernel for its shapes (D=128, Hkv=8, 4 or 8 query
    heads per kv head) in chunk mode with at most 64 chunks or, at 4, in
    balanced mode (a negative chunk_tiles) with at most 512 ranges, the MQA
    streaming kernel for one kv head at D=64, else the page-streaming kernel
    (always, with the page-kernel bit in the plan's wave count); other plans:
    the general kernel (its VALU-tile variant with the VALU bit)."""
    waves, page_bit, valu_bit = plan[2] & 0xFF, plan[2] & 0x100, plan[2] & 0x200
    balanced = plan[0] < 0
    if (waves == 16 and not page_bit and d == 128 and n_kv == 8 and (group == 4 or (group == 8 and not balanced))
            and plan[1] <= (512 if balanced else 64)):
        # (rocprofv3 prints this kernel mangled: _Float16 in its signature)
        return (f"_ZN4iris2st25int4_decode_stream_kernelILi8ELi{group}ELb{int(balanced)}EEEvPKiS3_PKDF16_"
                "iiiiiiiNS0_4ArgsE")
    if waves == 16 and not page_bit and n_kv == 1 and d == 64 and group <= 16:
        return "_ZN4iris2mq22int4_decode_mqa_kernelEPKiS2_PKDF16_iiiiiiNS0_4ArgsE"  # (printed mangled)
    if waves == 16:
        gs = 4
        while gs > 1 and gs * group > 16:
            gs //= 2
        gs = min(gs, d // 32)
        return f"void iris::pg::int4_decode_pages_kernel<{d}, {gs}, {n_kv}>(iris::pg::Args)"
    kvw = kernel_kvw(group, n_kv, batch, max_pages)
    if valu_bit:  # the VALU tile, measured against the MFMA one
        return f"void iris::int4_decode_valu_kernel<{d}, {kvw}>(iris::DecodeArgs)"
    return f"void iris::int4_decode_kernel<{d}, {kvw}>(iris::DecodeArgs)"


def kernel_kvw(group: int, n_kv: int, batch: int, max_pages: int) -> int:
    """KV heads per wavefront of the general decode kernel (as the library picks it:
    fewer while the grid would hold under 512 wave-tiles)."""
    kvw = 4
    while kvw > 1 and (kvw * group > 16 or n_kv % kvw):
        kvw //= 2
    cap_tiles = (max_pages * 16 + 31) // 32
    while kvw > 1 and batch * (cap_tiles + 1) * (n_kv // kvw) < 512:
        kvw //= 2
    return kvw


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5],
                    help="workload (2 is the metric's; others for analysis)")
    ap.add_argument("--replicas", type=int, default=0, help="cache copies to rotate (0 = auto)")
    ap.add_argument("--tokens-per-split", type=int, default=0)
    ap.add_argument("--waves-per-block", type=int, default=0)
    ap.add_argument("--decode-kernel", choices=["auto", "pages", "valu"], default="auto",
                    help="A/B runs: keep the page-streaming kernel for 16-wave plans (pages), or run the "
                         "general kernel's VALU tile (valu)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=0,
                    help="sequences in the CPU-baseline sample (0 = auto)")
    ap.add_argument("--no-bulk-append", action="store_true")
    ap.add_argument("--no-fp16", action="store_true", help="skip the matched FP16-cache decode leg")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 10 times (the reference kernel "
                         "whose FETCH_SIZE / WRITE_SIZE counters scale the decode kernel's)")
    ap.add_argument("--traffic", type=str, default=str(ROOT / "profiles" / "decode_cfg2_traffic.json"),
                    help="JSON with measured HBM bytes per decode launch (from rocprofv3 --pmc)")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def copy_calibration(torch, mib: int) -> int:
    """A device-to-device copy of exactly ``mib`` MiB (read once, written
    once), 10 launches: under ``rocprofv3 --pmc FETCH_SIZE`` (or
    WRITE_SIZE) its per-dispatch reading divided by ``mib`` * 1024 KiB is the
    counter's scale factor on this part."""
    dev = torch.device("cuda:0")
    n = mib * (1 << 20)
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(10):
        dst.copy_(src)
    ev[1].record()
    torch.cuda.synchronize()
    us = ev[0].elapsed_time(ev[1]) * 1e3 / 10
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "copy_us": round(us, 2),
                      "copy_gbs": round(2 * n / (us * 1e-6) / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path shards "
              "by kv head, or by page range with one all-gather of the fp32 partials per layer)", file=sys.stderr)
        return 2
    import torch

    if args.copy_calibration > 0:
        return copy_calibration(torch, args.copy_calibration)

    from iris_kernel import workloads
    from iris_kernel.fused_attention import _int4_paged_decode_attention, decode_plan
    from iris_kernel.fused_kv import _rope_int4_paged_append

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = workloads.CONFIGS[args.config]
    B, Hq, Hkv, D = cfg.batch, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim

    # ---------------------------------------------------------- workload
    t0 = time.time()
    case = workloads.decode_case(args.config)
    lens = case.seq_lens.tolist()
    cos, sin = case.cos.to(dev), case.sin.to(dev)
    cache0 = case.empty_cache(dev)
    # Prefill positions [0, L-1) with the fused append; the step appends L-1.
    case.fill_cache(lambda k, v, p, s, c, sn, *cc: _rope_int4_paged_append(k, v, p, s, c, sn, *cc, D, 16),
                    cache0, device=dev, upto=[n - 1 for n in lens])
    g = torch.Generator().manual_seed(workloads.SEED + 5)
    new_k = torch.randn((B, Hkv, D), generator=g).to(torch.float16).to(dev)
    new_v = torch.randn((B, Hkv, D), generator=g).to(torch.float16).to(dev)
    new_pos = (case.seq_lens - 1).to(torch.int32)
    new_slots = (case.block_table[torch.arange(B), (new_pos // 16).long()] * 16 + new_pos % 16).to(torch.int32)
    new_pos, new_slots = new_pos.to(dev), new_slots.to(dev)
    cache_bytes = sum(t.numel() * t.element_size() for t in cache0)
    reps = args.replicas or max(1, math.ceil(600e6 / cache_bytes))
    caches = [cache0] + [tuple(t.clone() for t in cache0) for _ in range(reps - 1)]
    q, bt, sl = (t.to(dev) for t in (case.query, case.block_table, case.seq_lens))
    out = torch.empty(q.shape, dtype=torch.float16, device=dev)
    from iris_kernel.fused_attention import DECODE_PAGE_KERNEL, DECODE_VALU_TILE

    select = {"auto": 0, "pages": DECODE_PAGE_KERNEL, "valu": DECODE_VALU_TILE}[args.decode_kernel]
    plan = decode_plan(B, Hq, Hkv, D, bt.shape[1], sum(lens), max(lens), args.tokens_per_split,
                       args.waves_per_block | select)
    ws = torch.zeros(max(plan[3], 1), dtype=torch.uint8, device=dev)  # counters start at zero
    torch.cuda.synchronize()
    log(f"config {args.config}: B={B} Hq={Hq} Hkv={Hkv} D={D} max L={max(lens)}; {reps} cache replicas of "
        f"{cache_bytes / 1e6:.1f} MB; plan chunk_tiles={plan[0]} max_chunks={plan[1]} waves={plan[2]}; "
        f"setup {time.time() - t0:.1f}s")

    from iris_kernel import fused_attention as fa

    def do_append(r):
        _rope_int4_paged_append(new_k, new_v, new_pos, new_slots, cos, sin, *caches[r], D, 16)

    def do_decode(r):
        fa._launch_decode(q, *caches[r], bt, sl, out, D ** -0.5, plan, ws)

    # ------------------------------------------- contract pass (wall clock)
    for i in range(args.warmup):
        do_append(i % reps)
        do_decode(i % reps)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(args.steps):
        do_append(i % reps)
        do_decode(i % reps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    ms_per_step = wall * 1e3 / args.steps

    # ------------------------------------ per-op pass (events around each op)
    n = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n)]
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e6) * n)  # keep the GPU busy while the host queues the n steps
    for i in range(n):
        r = i % reps
        ev[i][0].record()
        do_append(r)
        ev[i][1].record()
        ev[i][2].record()
        do_decode(r)
        ev[i][3].record()
    torch.cuda.synchronize()
    app_us = [e[0].elapsed_time(e[1]) * 1e3 for e in ev]
    dec_op_us = [e[2].elapsed_time(e[3]) * 1e3 for e in ev]
    app_mean = statistics.fmean(app_us)

    # --------------------------- decode kernel pass (back-to-back launches)
    # One event pair on the launch stream around n decodes that rotate over
    # the cache replicas: the average launch duration of the decode kernel
    # (what rocprofv3 --kernel-trace reports per dispatch), without the
    # per-event overhead of the pass above.
    def back_to_back(fn, n_reps):
        """Median over 3 passes of the mean launch duration (us) of n
        back-to-back calls of fn: each pass queues a GPU sleep (so the host
        enqueues every launch before the first runs), 5 untimed calls (the
        clocks back at load after the sleep), then the timed n."""
        k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        passes = []
        for _ in range(3):
            torch.cuda.synchronize()
            torch.cuda._sleep(int(1e6) * n)
            for i in range(5):
                fn(i % n_reps)
            k0.record()
            for i in range(n):
                fn(i % n_reps)
            k1.record()
            torch.cuda.synchronize()
            passes.append(k0.elapsed_time(k1) * 1e3 / n)
        return statistics.median(passes), passes

    dec_mean, dec_passes = back_to_back(do_decode, reps)
    dbytes = decode_bytes(B, Hq, Hkv, D, lens)
    abytes = append_bytes(B, Hkv, D, len(set(new_pos.tolist())))
    achieved = dbytes / (dec_mean * 1e-6) / 1e9
    log(f"decode: {dec_mean:.2f} us per launch back to back (per-op events: mean {statistics.fmean(dec_op_us):.2f}, "
        f"p50 {statistics.median(dec_op_us):.2f}) -> {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of 8 TB/s); "
        f"append {app_mean:.2f} us; wall {ms_per_step * 1e3:.1f} us/step")

    result = {
        "metric": METRIC,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": f"config {args.config}: {cfg.description}; step = fused RoPE+INT4 append of "
                        f"{B} tokens + INT4 paged decode attention",
            "batch": B, "num_q_heads": Hq, "num_kv_heads": Hkv, "head_dim": D, "page_size": 16,
            "seq_len": max(lens), "total_tokens": sum(lens), "cache_replicas": reps,
            "split_plan": {"chunk_tiles": plan[0], "max_chunks": plan[1], "waves_per_block": plan[2]},
        },
        "storage": "int4 codes + fp16 group-32 scales; fp16 MFMA operands, fp32 accumulate",
        "decode_us": round(dec_mean, 3),
        "decode_us_passes": [round(x, 3) for x in dec_passes],
        "decode_us_per_op_event_p50": round(statistics.median(dec_op_us), 3),
        "decode_tokens_per_s": round(B / (dec_mean * 1e-6), 1),
        "decode_hbm_gbs": round(achieved, 1),
        "decode_hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
        "decode_algorithmic_bytes": dbytes,
        "append_tokens": B,
        "append_us": round(app_mean, 3),
        "append_tokens_per_s": round(B / (app_mean * 1e-6), 1),
        "append_algorithmic_bytes": abytes,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": decode_kernel_name(plan, Hq // Hkv, Hkv, D, B, bt.shape[1]),
            "algorithmic_bytes_per_launch": dbytes,
        },
    }
    tpath = Path(args.traffic)
    if args.config == 2 and tpath.exists():
        # Counters measured on another kernel say nothing about this one.
        try:
            tr = json.loads(tpath.read_text())
            if tr.get("kernel") == result["roofline"]["kernel"]:
                result["roofline"]["traffic"] = tr.get("hbm_bytes_per_launch")
                result["roofline"]["traffic_source"] = str(tpath.relative_to(ROOT))
        except (ValueError, OSError):
            pass

    # ------------------------------------------------ bulk append (cfg 5)
    if not args.no_bulk_append:
        ac = workloads.append_case(5)
        T = ac.key.shape[0]
        tensors = [t.to(dev) for t in (ac.key, ac.value, ac.positions, ac.slot_mapping, ac.cos, ac.sin)]
        pool = ac.empty_cache(dev, fill="zeros")
        # Copies of K and V (and of the written pool) past the 256 MB MALL,
        # rotated, so each launch reads and writes HBM.
        kv_bytes = 2 * tensors[0].numel() * 2
        breps = max(1, math.ceil(600e6 / kv_bytes))
        kvs = [(tensors[0], tensors[1])] + [(tensors[0].clone(), tensors[1].clone()) for _ in range(breps - 1)]
        pools = [pool] + [tuple(t.clone() for t in pool) for _ in range(breps - 1)]

        def do_bulk(i):
            k, v = kvs[i % breps]
            _rope_int4_paged_append(k, v, *tensors[2:], *pools[i % breps], 128, 16)

        for i in range(2 * breps):
            do_bulk(i)
        torch.cuda.synchronize()
        n_bulk = 20 * breps
        bev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda._sleep(int(2e6))  # the host queues every launch ahead of the GPU
        bev[0].record()
        for i in range(n_bulk):
            do_bulk(i)
        bev[1].record()
        torch.cuda.synchronize()
        bulk_us = bev[0].elapsed_time(bev[1]) * 1e3 / n_bulk
        bbytes = append_bytes(T, 8, 128, 8192)
        result["append_bulk"] = {
            "workload": "config 5 bulk append: 4 x 8192 tokens, Hkv=8, D=128, RoPE base 5e5",
            "tokens": T, "us": round(bulk_us, 2), "tokens_per_s": round(T / (bulk_us * 1e-6), 1),
            "replicas": breps, "timing": "back-to-back launches, one HIP event pair",
            "hbm_gbs": round(bbytes / (bulk_us * 1e-6) / 1e9, 1),
            "hbm_frac": round(bbytes / (bulk_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": bbytes,
        }
        log(f"bulk append: {bulk_us:.2f} us for {T} tokens -> {T / (bulk_us * 1e-6) / 1e6:.1f} M tok/s, "
            f"{bbytes / (bulk_us * 1e-6) / 1e9:.0f} GB/s")

    # ----------------------------- matched FP16-cache decode (reference's comparator)
    if not args.no_fp16:
        from iris_kernel.fused_attention import _fp16_paged_decode_attention
        from iris_kernel.fused_kv import _rope_fp16_paged_append

        shape16 = (case.num_pages, 16, Hkv, D)
        c16 = (torch.zeros(shape16, dtype=torch.float16, device=dev), torch.zeros(shape16, dtype=torch.float16, device=dev))
        case.fill_cache(lambda k, v, p_, s, c, sn, kc, vc: _rope_fp16_paged_append(k, v, p_, s, c, sn, kc, vc, D, D, 16),
                        c16, device=dev)
        reps16 = max(1, math.ceil(600e6 / (2 * c16[0].numel() * 2)))
        caches16 = [c16] + [tuple(t.clone() for t in c16) for _ in range(reps16 - 1)]
        out16 = torch.empty_like(out)

        def do_fp16(r):
            _fp16_paged_decode_attention(q, *caches16[r], bt, sl, out16, D, 16)

        for i in range(args.warmup):
            do_fp16(i % reps16)
        f16_us, f16_passes = back_to_back(do_fp16, reps16)
        f16_bytes = sum(lens) * Hkv * 4 * D + 2 * B * Hq * D * 2 + 4 * sum((x + 15) // 16 for x in lens) + 4 * B
        result["fp16_decode"] = {
            "workload": "same decode over an fp16 cache [NP, 16, Hkv, D] (the reference's matched FP16 baseline)",
            "us": round(f16_us, 3), "algorithmic_bytes": f16_bytes,
            "hbm_gbs": round(f16_bytes / (f16_us * 1e-6) / 1e9, 1),
            "hbm_frac": round(f16_bytes / (f16_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "int4_speedup": round(f16_us / dec_mean, 3), "cache_replicas": reps16,
            "us_passes": [round(x, 3) for x in f16_passes],
        }
        log(f"fp16 decode: {f16_us:.2f} us ({f16_bytes / (f16_us * 1e-6) / 1e9:.0f} GB/s); INT4 is "
            f"{f16_us / dec_mean:.2f}x faster")
        del caches16, c16

    # ------------------------------------------------ CPU baseline (port)
    if not args.no_cpu_baseline:
        from oracle.torch_eager_attention import torch_eager_int4_paged_decode_attention
        from oracle.torch_eager_kv import torch_eager_append

        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        cpu_cache = tuple(t.cpu() for t in caches[0])

        def timed(fn, runs=5, budget_s=8.0):
            fn()  # warm-up
            times, t_end = [], time.perf_counter() + budget_s
            for _ in range(runs):
                t1 = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t1)
                if time.perf_counter() > t_end:
                    break
            return statistics.median(times), len(times)

        # decode: as many of the B sequences as ~2 s a run allows (at least 4)
        t1 = time.perf_counter()
        torch_eager_int4_paged_decode_attention(case.query[:1], *cpu_cache, case.block_table[:1], case.seq_lens[:1])
        per_seq = time.perf_counter() - t1
        sample = args.cpu_sample or max(4, min(B, int(2.0 / max(per_seq, 1e-6))))
        q_s, bt_s, sl_s = case.query[:sample], case.block_table[:sample], case.seq_lens[:sample]
        ref = None

        def cpu_decode():
            nonlocal ref
            ref = torch_eager_int4_paged_decode_attention(q_s, *cpu_cache, bt_s, sl_s)

        cpu_s, n_dec = timed(cpu_decode)
        sbytes = decode_bytes(sample, Hq, Hkv, D, lens[:sample])
        # the GPU output of the last decode on replica 0 for the same sequences
        do_decode(0)
        torch.cuda.synchronize()
        err = (out[:sample].float().cpu() - ref.float()).abs().max().item()

        # append, the step's: one new token per sequence into the cache
        step_args = [t.cpu() for t in (new_k, new_v, new_pos, new_slots, cos, sin)]
        app_cpu_s, n_app = timed(lambda: torch_eager_append(*step_args, *cpu_cache, rotary_dim=D, group_size=32,
                                                            page_size=16), runs=20)
        # bulk append (configuration 5), a bounded sample of its tokens
        ac = workloads.append_case(5)
        bulk_n = min(ac.key.shape[0], 4096)
        bpool = ac.empty_cache(torch.device("cpu"), fill="zeros")
        bargs = (ac.key[:bulk_n], ac.value[:bulk_n], ac.positions[:bulk_n], ac.slot_mapping[:bulk_n], ac.cos, ac.sin)
        bulk_cpu_s, n_bulk_cpu = timed(lambda: torch_eager_append(*bargs, *bpool, rotary_dim=128, group_size=32,
                                                                  page_size=16))
        cpu_model = "unknown"
        try:
            for line in Path("/proc/cpuinfo").read_text().splitlines():
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
        result["cpu_baseline"] = {
            "value": round(sbytes / cpu_s / 1e9, 3),
            "unit": "GB/s",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "cpu_model": cpu_model,
            "sample": f"decode of the first {sample} of {B} sequences (L={lens[0]}) with the torch "
                      f"restatement of torch_eager_int4_paged_decode_attention, median of {n_dec} runs "
                      f"= {cpu_s * 1e3:.1f} ms; append: the step's {B}-token append (median of {n_app} runs) "
                      f"and the first {bulk_n} of configuration 5's {ac.key.shape[0]} bulk-append tokens "
                      f"(median of {n_bulk_cpu}), with the restatement of torch_eager_append",
            "decode_us_equiv_full_batch": round(cpu_s * 1e6 * B / sample, 1),
            "gpu_vs_eager_max_abs_err": err,
            "append_tokens_per_s": round(B / app_cpu_s, 1),
            "append_us": round(app_cpu_s * 1e6, 1),
            "bulk_append_tokens_per_s": round(bulk_n / bulk_cpu_s, 1),
        }
        log(f"cpu baseline ({cpu_model}, {threads} threads): decode {sbytes / cpu_s / 1e9:.3f} GB/s "
            f"({sample} sequences), append {B / app_cpu_s:.0f} tok/s, bulk append {bulk_n / bulk_cpu_s:.0f} tok/s; "
            f"GPU vs eager max-abs err {err:.2e}")

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
