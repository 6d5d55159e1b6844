#!/usr/bin/env python3
"""INT4 decode at head_dim 96, 160, 192 and 224 on MI355X: the MFMA kernel
of csrc/decode_hd.hip (the plan's choice) against the any-shape kernel of
csrc/decode_any.hip (IRIS_DECODE_ANY_KERNEL), per shape.

Each shape is (B, Hq, Hkv, D, L[, ragged]): B sequences of L tokens (ragged:
lengths log-uniform in [128, L]), 16-token pages in a shuffled block table,
random codes and scales in [0.05, 0.25].  The cache is replicated past the
256 MB last-level cache and the copies rotated, so every launch reads HBM.
Each kernel's launches are timed one at a time with HIP events (median of
``--n``); the two outputs are compared before timing.  The algorithmic
bytes are the K and V codes and scales of the valid tokens, the query and
the output: (D + D / 8) bytes a token and kv head.

Run: python tests/bench_head_dims.py [--n 30] [--shapes "8,32,8,96,8192;..."] [--json out.json]
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

from iris_kernel.fused_attention import DECODE_ANY_KERNEL, _launch_decode, int4_decode_plan  # noqa: E402

SHAPES = [
    (8, 32, 8, 96, 8192), (32, 32, 8, 96, 4096), (128, 16, 1, 96, 8192), (16, 40, 8, 96, 8192),
    (8, 32, 8, 160, 8192), (4, 64, 8, 160, 32768),
    (8, 32, 8, 192, 8192), (32, 32, 8, 192, 4096),
    (8, 32, 8, 224, 8192), (64, 32, 8, 224, 4096, 1),
]


def run_shape(dev, shape, n):
    B, Hq, Hkv, D, L = shape[:5]
    ragged = len(shape) > 5 and shape[5]
    g = torch.Generator().manual_seed(B + D)
    if ragged:
        lens = torch.exp(torch.empty(B).uniform_(math.log(128), math.log(L), generator=g)).long().clamp(1, L)
    else:
        lens = torch.full((B,), L, dtype=torch.long)
    cols = -(-L // 16)
    num_pages = B * cols + 1
    bt = torch.randperm(num_pages, generator=g)[: B * cols].view(B, cols).to(torch.int32).to(dev)
    sl = lens.to(torch.int32).to(dev)
    copies = max(1, math.ceil(800e6 / (num_pages * 16 * Hkv * (D + D // 8))))
    gd = torch.Generator(device=dev).manual_seed(1)
    caches = [(torch.randint(0, 256, (num_pages, 16, Hkv, D // 2), dtype=torch.uint8, device=dev, generator=gd),
               torch.randint(0, 256, (num_pages, 16, Hkv, D // 2), dtype=torch.uint8, device=dev, generator=gd),
               (torch.rand(num_pages, 16, Hkv, D // 32, device=dev, generator=gd) * 0.2 + 0.05).half(),
               (torch.rand(num_pages, 16, Hkv, D // 32, device=dev, generator=gd) * 0.2 + 0.05).half())
              for _ in range(copies)]
    q = torch.randn(B, Hq, D, device=dev, generator=gd).half()
    total = int(lens.sum())
    algo = total * Hkv * (D + D // 8) + 2 * B * Hq * D * 2
    row = {"B": B, "Hq": Hq, "Hkv": Hkv, "D": D, "L": L, "ragged": bool(ragged), "bytes": algo}
    outs = {}
    for name, wpb in (("hd", 0), ("any", DECODE_ANY_KERNEL)):
        plan = int4_decode_plan(B, Hq, Hkv, D, 16, cols, total, int(lens.max()), 0, wpb)
        out = torch.empty(B, Hq, D, dtype=torch.float32, device=dev)

        def launch(r, plan=plan, out=out):
            _launch_decode(q, *caches[r], bt, sl, out, D ** -0.5, plan)

        for r in range(copies):
            launch(r)
        torch.cuda.synchronize()
        outs[name] = out.clone()
        times = []
        for i in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch(i % copies)
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1000.0)
        times.sort()
        us = times[len(times) // 2]
        row[name] = {"us": round(us, 2), "TB/s": round(algo / us / 1e6, 3), "plan": list(plan)}
    row["max_abs_diff"] = (outs["hd"] - outs["any"]).abs().max().item()
    assert row["max_abs_diff"] < 2e-3, row
    del caches
    torch.cuda.empty_cache()
    return row


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, default=30)
    ap.add_argument("--shapes", type=str, default="", help='"B,Hq,Hkv,D,L[,ragged];..."')
    ap.add_argument("--json", type=str, default="")
    args = ap.parse_args()
    shapes = [tuple(int(x) for x in s.split(",")) for s in args.shapes.split(";")] if args.shapes else SHAPES
    dev = torch.device("cuda:0")
    rows = []
    print("| B | Hq | Hkv | D | L | MB | head-dim kernel µs | TB/s | any-shape kernel µs | TB/s | speed-up |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for shape in shapes:
        r = run_shape(dev, shape, args.n)
        rows.append(r)
        L = f"{r['L']} ragged" if r["ragged"] else str(r["L"])
        print(f"| {r['B']} | {r['Hq']} | {r['Hkv']} | {r['D']} | {L} | {r['bytes'] / 1e6:.0f} | {r['hd']['us']:.1f} | "
              f"{r['hd']['TB/s']:.2f} | {r['any']['us']:.1f} | {r['any']['TB/s']:.2f} | "
              f"{r['any']['us'] / r['hd']['us']:.2f}x |", flush=True)
    if args.json:
        Path(args.json).write_text(json.dumps(rows, indent=1))


if __name__ == "__main__":
    main()
