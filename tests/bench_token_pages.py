#!/usr/bin/env python3
"""INT4 decode on the token-page mode of csrc/decode_hd.hip
(IRIS_DECODE_TOKEN_PAGES: each token's page looked up through the block
table, any page size) against the other kernels that take the same shape:
the any-shape kernel (IRIS_DECODE_ANY_KERNEL) at every page size, and, at
16-token pages and head_dim 64 or 128, the general kernel (4 waves) and the
plan's own choice.

Each shape is (B, Hq, Hkv, D, L, P[, ragged]): B sequences of L tokens
(ragged: lengths log-uniform in [16, L]), P-token pages in a shuffled block
table, random codes and scales in [0.05, 0.25].  The cache is replicated
past the 256 MB last-level cache and the copies rotated, so every launch
reads HBM.  Each kernel is timed with HIP events around ``--n``
back-to-back launches (so the host's time to issue a launch overlaps the
previous one), the median over ``--batches`` such batches; the outputs are
compared with the token-page mode's before timing.  The algorithmic bytes
are the K and V codes and scales of the valid tokens, the query and the
output: (D + D / 8) bytes a token and kv head.

Run: python tests/bench_token_pages.py [--n 20] [--batches 5] [--shapes "8,32,8,128,8192,8;..."] [--no-any] [--json out.json]
"""
from __future__ import annotations

import argparse
import json
import math
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "iris-kernel_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

from iris_kernel.fused_attention import (DECODE_ANY_KERNEL, DECODE_TOKEN_PAGES, _launch_decode,  # noqa: E402
                                         int4_decode_plan)

SHAPES = [
    (8, 32, 8, 128, 8192, 8), (32, 32, 8, 128, 4096, 24), (128, 16, 1, 64, 8192, 8), (8, 32, 8, 96, 8192, 24),
    (8, 32, 8, 192, 8192, 1), (4, 32, 8, 128, 32768, 40), (8, 32, 8, 224, 8192, 12),
    (1, 32, 8, 128, 4096, 16), (4, 32, 8, 128, 8192, 16), (8, 32, 8, 128, 8192, 16), (32, 32, 8, 128, 2048, 16),
    (1, 32, 8, 128, 32768, 16), (32, 32, 8, 64, 2048, 16), (64, 8, 2, 64, 2048, 16), (32, 128, 8, 128, 2048, 16),
]


def run_shape(dev, shape, n, batches, with_any):
    B, Hq, Hkv, D, L, P = shape[:6]
    ragged = len(shape) > 6 and shape[6]
    g = torch.Generator().manual_seed(B + D + P)
    if ragged:
        lens = torch.exp(torch.empty(B).uniform_(math.log(16), math.log(L), generator=g)).long().clamp(1, L)
    else:
        lens = torch.full((B,), L, dtype=torch.long)
    cols = -(-L // P)
    num_pages = B * cols + 1
    bt = torch.randperm(num_pages, generator=g)[: B * cols].view(B, cols).to(torch.int32).to(dev)
    sl = lens.to(torch.int32).to(dev)
    copies = max(1, math.ceil(800e6 / (num_pages * P * Hkv * (D + D // 8))))
    gd = torch.Generator(device=dev).manual_seed(1)
    caches = [(torch.randint(0, 256, (num_pages, P, Hkv, D // 2), dtype=torch.uint8, device=dev, generator=gd),
               torch.randint(0, 256, (num_pages, P, Hkv, D // 2), dtype=torch.uint8, device=dev, generator=gd),
               (torch.rand(num_pages, P, Hkv, D // 32, device=dev, generator=gd) * 0.2 + 0.05).half(),
               (torch.rand(num_pages, P, Hkv, D // 32, device=dev, generator=gd) * 0.2 + 0.05).half())
              for _ in range(copies)]
    q = torch.randn(B, Hq, D, device=dev, generator=gd).half()
    total = int(lens.sum())
    algo = total * Hkv * (D + D // 8) + 2 * B * Hq * D * 2
    row = {"B": B, "Hq": Hq, "Hkv": Hkv, "D": D, "L": L, "P": P, "ragged": bool(ragged), "bytes": algo}
    kernels = [("tok", DECODE_TOKEN_PAGES)]
    if with_any:
        kernels.append(("any", DECODE_ANY_KERNEL))
    if P % 16 == 0 and D in (64, 128):
        kernels += [("general", 4), ("plan", 0)]
    outs = {}
    for name, wpb in kernels:
        plan = int4_decode_plan(B, Hq, Hkv, D, P, cols, total, int(lens.max()), 0, wpb)
        if name == "tok":
            assert plan[2] & DECODE_TOKEN_PAGES, plan
        out = torch.empty(B, Hq, D, dtype=torch.float32, device=dev)

        def launch(r, plan=plan, out=out):
            _launch_decode(q, *caches[r], bt, sl, out, D ** -0.5, plan)

        for r in range(copies):
            launch(r)
        torch.cuda.synchronize()
        outs[name] = out.clone()
        times = []
        for b in range(batches):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(n):
                launch((b * n + i) % copies)
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1000.0 / n)
        times.sort()
        us = times[len(times) // 2]
        row[name] = {"us": round(us, 2), "TB/s": round(algo / us / 1e6, 3), "plan": list(plan)}
    for name in outs:
        diff = (outs[name] - outs["tok"]).abs().max().item()
        assert diff < 2e-3, (name, diff, row)
    del caches
    torch.cuda.empty_cache()
    return row


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, default=20, help="back-to-back launches a timed batch")
    ap.add_argument("--batches", type=int, default=5)
    ap.add_argument("--shapes", type=str, default="", help='"B,Hq,Hkv,D,L,P[,ragged];..."')
    ap.add_argument("--no-any", action="store_true", help="leave out the any-shape kernel")
    ap.add_argument("--json", type=str, default="")
    args = ap.parse_args()
    shapes = [tuple(int(x) for x in s.split(",")) for s in args.shapes.split(";")] if args.shapes else SHAPES
    dev = torch.device("cuda:0")
    rows = []
    print("| B | Hq | Hkv | D | L | P | MB | token pages µs | TB/s | any-shape µs | general µs | plan's choice µs |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|")
    for shape in shapes:
        r = run_shape(dev, shape, args.n, args.batches, not args.no_any)
        rows.append(r)
        L = f"{r['L']} ragged" if r["ragged"] else str(r["L"])
        cell = lambda k: f"{r[k]['us']:.1f}" if k in r else "-"  # noqa: E731
        plan = f"{r['plan']['us']:.1f} ({r['plan']['plan'][2]:#x})" if "plan" in r else "-"
        print(f"| {r['B']} | {r['Hq']} | {r['Hkv']} | {r['D']} | {L} | {r['P']} | {r['bytes'] / 1e6:.0f} | "
              f"{r['tok']['us']:.1f} | {r['tok']['TB/s']:.2f} | {cell('any')} | {cell('general')} | {plan} |",
              flush=True)
    if args.json:
        Path(args.json).write_text(json.dumps(rows, indent=1))


if __name__ == "__main__":
    main()
