"""The balanced splits of ragged batches restated in Python and checked for
the properties their merges and memory safety rest on, over random ragged
batches and the plans iris_decode_plan makes for them.

* The page kernel's (decode_pages.hip, balanced mode): W range workgroups
  and B sequence-start workgroups, one segment each.
* The streaming kernel's (decode_stream.hip, balanced mode): W ranges of
  cost units (every sequence's tiles plus kPieceCost), one workgroup each,
  walking every piece its range meets.

Properties: every tile of every sequence is in exactly one piece; each
(sequence, chunk) has a slot w + b < W + B of its own; chunk indices of a
sequence run 0 .. n_chunks - 1 over consecutive ranges; no piece exceeds the
64-tile page-id window; a range meets at most kMaxPieces pieces (the
streaming kernel's LDS list).  Runs without a GPU.
"""
import random

import pytest

from iris_kernel.fused_attention import DECODE_PAGE_KERNEL, decode_plan

PIECE_COST = 5   # kPieceCost of csrc/decode_stream.hip
MAX_PIECES = 40  # kMaxPieces of csrc/decode_stream.hip


def segments(lens, W):
    """(workgroup, b, t_begin, t_end, c, n_chunks, first) for every workgroup
    that has a segment, as the kernel's balanced mode finds them."""
    n = [max(0, (L + 31) // 32) for L in lens]
    T = sum(n)
    P = [0]
    for x in n:
        P.append(P[-1] + x)
    if T == 0:
        return []
    Wg, W = W, min(W, T)  # W range workgroups at most T ranges (Wg launched)
    lo = lambda w: w * T // W  # noqa: E731
    hi = lambda w: min((w + 1) * T // W, lo(w) + 64)  # noqa: E731
    out = []
    for bid in range(Wg + len(lens)):
        for b, nb in enumerate(n):
            if nb == 0:
                continue
            pb = P[b]
            w = -1
            if bid < Wg:
                if bid < W and pb <= lo(bid) < pb + nb and lo(bid) < hi(bid):
                    w = bid
            elif b == bid - Wg:
                f = ((pb + 1) * W - 1) // T
                if lo(f) < pb < hi(f):
                    w = f
            if w >= 0:
                f, last = ((pb + 1) * W - 1) // T, ((pb + nb) * W - 1) // T
                out.append((bid, b, max(lo(w), pb) - pb, min(hi(w), pb + nb) - pb, w - f, last - f + 1, f))
    return out


def check(lens, W):
    segs = segments(lens, W)
    n = [max(0, (L + 31) // 32) for L in lens]
    assert len({s[0] for s in segs}) == len(segs), "one segment per workgroup"
    covered = {}
    slots = set()
    chunks = {}
    for bid, b, t0, t1, c, nch, first in segs:
        assert 0 <= t0 < t1 <= n[b] and t1 - t0 <= 64
        for t in range(t0, t1):
            assert (b, t) not in covered, "tile twice"
            covered[(b, t)] = bid
        slot = first + c + b
        assert slot < W + len(lens) and slot not in slots
        slots.add(slot)
        chunks.setdefault(b, []).append((c, nch, t0, t1))
    T = sum(n)
    if T == 0 or -(-T // W) > 64:
        return  # a grid the plans never make: memory-safe, tiles past a range's 64 dropped
    assert len(covered) == T, "every tile once"
    for b, cs in chunks.items():
        cs.sort()
        assert [c for c, *_ in cs] == list(range(len(cs))) and all(nch == len(cs) for _, nch, *_ in cs)
        assert cs[0][2] == 0 and cs[-1][3] == n[b]
        assert all(cs[i][3] == cs[i + 1][2] for i in range(len(cs) - 1)), "chunks in order, no gap"


@pytest.mark.parametrize("seed", range(40))
def test_random_ragged_batches(seed):
    rng = random.Random(seed)
    B = rng.choice([1, 2, 3, 7, 64, 130, 500])
    kind = seed % 4
    if kind == 0:
        lens = [int(round(2 ** rng.uniform(7, 14))) for _ in range(B)]  # log-uniform, configuration 3's law
    elif kind == 1:
        lens = [rng.randint(1, 40) for _ in range(B)]  # many sequences per range
    elif kind == 2:
        lens = [rng.choice([1, 16, 17, 31, 32, 33, 4096]) for _ in range(B)]
    else:
        lens = [rng.randint(1, 20000) for _ in range(B)]
    W = rng.choice([1, 2, 8, 31, 64, 255, 256, 512])
    check(lens, W)


@pytest.mark.parametrize("lens", [
    [16384] + [128] * 63,
    [1] * 299 + [40],
    [100000, 7, 100000],
    [int(round(2 ** (7 + 7 * i / 63))) for i in range(64)],
])
def test_planned_grids(lens):
    # the plan's W for these lengths keeps every share within 64 tiles
    B = len(lens)
    max_pages = (max(lens) + 15) // 16
    share, W, nw, ws = decode_plan(B, 32, 8, 128, max_pages, sum(lens), max(lens),
                                   waves_per_block=16 | DECODE_PAGE_KERNEL)
    assert share < 0 and nw == 16 | DECODE_PAGE_KERNEL
    T = sum((L + 31) // 32 for L in lens)
    assert -(-T // W) <= -share <= 64
    check(lens, W)
    # the streaming kernel's plan for the same batch (its shape: Hq 32, Hkv 8, D 128)
    share, W, nw, ws = decode_plan(B, 32, 8, 128, max_pages, sum(lens), max(lens), waves_per_block=16)
    assert share < 0 and nw == 16 and W <= 256
    C = sum((L + 31) // 32 + PIECE_COST for L in lens)
    assert -(-C // W) <= -share <= 64
    assert check_stream(lens, W) == "ok"


def stream_pieces(lens, W, cost=PIECE_COST):
    """(w, b, t_begin, t_end, c, n_chunks, first) for every piece, as the
    streaming kernel's balanced mode finds them; None where the kernel
    poisons the output (ranges longer than the 64-tile window)."""
    n = [max(0, (L + 31) // 32) for L in lens]
    U = [x + cost if x > 0 else 0 for x in n]
    C = sum(U)
    if C == 0:
        return []
    Wl = min(W, C)
    if C > 64 * Wl:
        return None
    S = [0]
    for u in U:
        S.append(S[-1] + u)
    range_of = lambda u: ((u + 1) * Wl - 1) // C  # noqa: E731
    out = []
    for w in range(Wl):
        lo, hi = w * C // Wl, (w + 1) * C // Wl
        for b in range(len(lens)):
            if U[b] == 0:
                continue
            ts, te = S[b] + cost, S[b] + U[b]
            if ts < hi and te > lo:
                f, last = range_of(ts), range_of(te - 1)
                out.append((w, b, max(lo, ts) - ts, min(hi, te) - ts, w - f, last - f + 1, f))
    return out


def check_stream(lens, W):
    pieces = stream_pieces(lens, W)
    if pieces is None:
        return "poisoned"
    n = [max(0, (L + 31) // 32) for L in lens]
    per_range = {}
    covered, slots, chunks = set(), set(), {}
    for w, b, t0, t1, c, nch, first in pieces:
        per_range[w] = per_range.get(w, 0) + 1
        assert 0 <= t0 < t1 <= n[b] and t1 - t0 <= 64
        for t in range(t0, t1):
            assert (b, t) not in covered, "tile twice"
            covered.add((b, t))
        slot = first + b + c
        assert slot == w + b and slot < W + len(lens) and slot not in slots
        slots.add(slot)
        chunks.setdefault(b, []).append((c, nch, t0, t1))
    assert max(per_range.values(), default=0) <= MAX_PIECES
    assert len(covered) == sum(n), "every tile once"
    for b, cs in chunks.items():
        cs.sort()
        assert [c for c, *_ in cs] == list(range(len(cs))) and all(nch == len(cs) for _, nch, *_ in cs)
        assert cs[0][2] == 0 and cs[-1][3] == n[b]
        assert all(cs[i][3] == cs[i + 1][2] for i in range(len(cs) - 1)), "chunks in order, no gap"
    return "ok"


@pytest.mark.parametrize("seed", range(40))
def test_stream_split_random_ragged_batches(seed):
    rng = random.Random(1000 + seed)
    B = rng.choice([1, 2, 3, 7, 64, 130, 500])
    kind = seed % 4
    if kind == 0:
        lens = [int(round(2 ** rng.uniform(7, 14))) for _ in range(B)]
    elif kind == 1:
        lens = [rng.randint(1, 40) for _ in range(B)]  # many sequences per range
    elif kind == 2:
        lens = [rng.choice([1, 16, 17, 31, 32, 33, 4096]) for _ in range(B)]
    else:
        lens = [rng.randint(1, 20000) for _ in range(B)]
    W = rng.choice([1, 2, 8, 31, 64, 255, 256, 512])
    check_stream(lens, W)


def test_stream_split_poisons_only_outgrown_plans():
    # a plan for 40-token sequences, lengths grown to 4096: past the window
    lens = [40] * 31 + [70]
    share, W, nw, ws = decode_plan(32, 32, 8, 128, 256, sum(lens), max(lens), waves_per_block=16)
    assert check_stream(lens, W) == "ok"
    assert check_stream([4096] * 32, W) == "poisoned"
