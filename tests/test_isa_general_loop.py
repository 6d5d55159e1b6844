"""The general decode kernel's tile loop, checked in its compiled gfx950 code.

The loop keeps the next tile's loads in flight while the current tile is
computed, which holds only if the compiler adds no wait of its own inside the
loop and builds every buffer descriptor from wave-uniform values.  Two
regressions this guards against, both seen in earlier builds of decode.hip:
a vmcnt(0) before each transposed V read (the compiler could not tell those
reads from the next tile's direct-to-LDS loads), and a loop of
v_readfirstlane around every K load (a descriptor word kept in a VGPR).
Compiles decode.hip once (about half a minute); runs without a GPU."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from iris_kernel import _build

SRC = _build.CSRC / "decode.hip"


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    try:
        hipcc = _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if shutil.which(hipcc) is None and not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "decode.s"
    cmd = [hipcc, *_build._common_flags(), "--cuda-device-only", "-S", str(SRC), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def tile_loop(asm: str, symbol: str) -> list[str]:
    """Instructions of the kernel's first outermost loop (the tile loop: the
    blocks the compiler annotates with its header, and loops nested in it)."""
    body = asm[asm.index(symbol + ":"):]
    body = body[:body.index(".Lfunc_end")]
    lines = [l.strip() for l in body.split("\n")]
    header = next(re.match(r"^\.LBB(\d+_\d+):", l).group(1) for l in lines if "Loop Header: Depth=1" in l)
    out, inside = [], False
    for l in lines:
        if re.match(r"^\.LBB\d+_\d+:", l) or l.startswith("; %bb"):
            inside = (l.startswith(f".LBB{header}:") or f"Header=BB{header} " in l + " "
                      or f"Parent Loop BB{header} " in l + " ")  # inner loops too
            continue
        if inside and l and not l.startswith(";"):
            out.append(l)
    return out


def symbols(asm: str) -> list[str]:
    return re.findall(r"^(_ZN4iris18int4_decode_kernelILi(\d+)ELi(\d)E\w+):", asm, flags=re.M)


def test_every_layout_is_compiled(asm):
    assert sorted((int(d), int(k)) for _, d, k in symbols(asm)) == [(64, 1), (64, 2), (64, 4),
                                                                    (128, 1), (128, 2), (128, 4),
                                                                    (256, 1)]


def test_tile_loop_waits_only_at_the_tile_boundary(asm):
    for sym, d, _ in symbols(asm):
        loop = tile_loop(asm, sym)
        assert sum(1 for l in loop if l.startswith("v_mfma")) >= 16, sym  # the loop found is the tile loop
        assert sum(1 for l in loop if l.startswith("ds_read_b64_tr_b8")) >= 4, sym
        waits = [l for l in loop if l.startswith("s_waitcnt") and "vmcnt" in l]
        assert all("vmcnt(0)" in w for w in waits), (sym, waits)
        # one wait per tile (the loop body holds two tiles); at D = 128 the
        # compiler adds one before the last PV products of the second tile
        assert len(waits) <= (2 if d == "64" else 4), (sym, waits)


def test_no_waterfall_loop_around_loads(asm):
    for sym, _, _ in symbols(asm):
        loop = tile_loop(asm, sym)
        assert not [l for l in loop if l.startswith("v_readfirstlane")], sym
        assert not [l for l in loop if l.startswith("scratch_")], sym  # no spills in the loop either
