"""The head_dim 96-224 decode kernel's tile loop, checked in its compiled
gfx950 code (csrc/decode_hd.hip, every G instance of both modes: pages of
16 m tokens, and token pages at head_dim 64-256, with the per-token scale
shifts of odd scale rows at G = 3, 5, 7).

A wave keeps the next tile's direct-to-LDS loads in flight while it
computes one, which holds only if every vmcnt wait in the loop is one of the
kernel's own (one tile's load instructions or none, plus, in token-page
mode, the one load of a tile's block-table entries: the compiler would
otherwise wait for the loads streaming into the other slot).  Two
regressions this guards against, both seen while the kernel was written: the
loop compiled as a divergent loop (its bounds in VGPRs, an exec-mask exit
around every tile), and spilled registers.  Compiles decode_hd.hip once
(a few seconds); runs without a GPU."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from iris_kernel import _build

SRC = _build.CSRC / "decode_hd.hip"
GROUPS = [3, 5, 6, 7]  # head_dim / 32
# (G, token pages, per-token scale shifts)
INSTANCES = ([(g, False, False) for g in GROUPS] + [(g, True, False) for g in (2, 3, 4, 5, 6, 7, 8)]
             + [(g, True, True) for g in (3, 5, 7)])


def jobs_of(g: int, tok: bool) -> int:
    """Load instructions of one tile: 16-byte code loads (32 g pieces of 64
    lanes) and 4-byte scale loads (2 or 4 dwords a token: g halves from the
    first, on the second half of a dword only where g is odd), for K and V;
    at g = 2 and 8 in token-page mode one 4- or 16-byte load a token for
    both scale tensors."""
    sd = (g + (g & 1)) // 2
    sp = 1 if sd <= 1 else 2 if sd <= 2 else 4
    scale_jobs = 1 if (tok and g in (2, 8)) else 2 * ((32 * sp + 63) // 64)
    return 2 * ((32 * g + 63) // 64) + scale_jobs


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    try:
        hipcc = _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if shutil.which(hipcc) is None and not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "decode_hd.s"
    cmd = [hipcc, *_build._common_flags(), *_build.SOURCES["decode_hd.hip"], "--cuda-device-only", "-S",
           str(SRC), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def kernel(asm: str, g: int, tok: bool, odd: bool) -> list[str]:
    sym = f"_ZN4iris2hd21int4_decode_hd_kernelILi{g}ELb{int(tok)}ELb{int(odd)}EEEvNS0_4ArgsE"
    body = asm[asm.index(sym + ":"):]
    body = body[:body.index(".Lfunc_end")]
    return [l.strip() for l in body.split("\n")]


def tile_loop(lines: list[str]) -> list[str]:
    """Instructions of the kernel's first outermost loop (the tile loop)."""
    header = next(re.match(r"^\.LBB(\d+_\d+):", l).group(1) for l in lines if "Loop Header: Depth=1" in l)
    out, inside = [], False
    for l in lines:
        if re.match(r"^\.LBB\d+_\d+:", l) or l.startswith("; %bb"):
            inside = (l.startswith(f".LBB{header}:") or f"Header=BB{header} " in l + " "
                      or f"Parent Loop BB{header} " in l + " ")
            continue
        if inside and l and not l.startswith(";"):
            out.append(l)
    return out


@pytest.mark.parametrize("g,tok,odd", INSTANCES)
def test_tile_loop_is_the_tile_loop(asm, g, tok, odd):
    loop = tile_loop(kernel(asm, g, tok, odd))
    # per tile: 2 G QK and 2 G PV products, G transposed V reads
    assert sum(1 for l in loop if l.startswith("v_mfma")) == 4 * g
    assert sum(1 for l in loop if l.startswith("ds_read_b64_tr_b8")) == g


@pytest.mark.parametrize("g,tok,odd", INSTANCES)
def test_tile_loop_waits_only_for_its_own_tiles(asm, g, tok, odd):
    loop = tile_loop(kernel(asm, g, tok, odd))
    jobs = jobs_of(g, tok)
    loads = sum(1 for l in loop if l.startswith("global_load_lds"))
    waits = {int(m) for l in loop if l.startswith("s_waitcnt") for m in re.findall(r"vmcnt\((\d+)\)", l)}
    # one tile in flight while one is computed (the last tile's vmcnt(0) may
    # sit in the loop or in its peeled last iteration)
    assert jobs in waits, (jobs, sorted(waits))
    if not tok:
        assert loads == jobs, (loads, jobs)  # one tile's loads, issued once a step
        assert all(w % jobs == 0 and w < 64 for w in waits), (jobs, sorted(waits))
    else:
        # a tile's data loads (in one or two copies of the issue) and the
        # next entries' one load; waits for a tile or a tile and the entries
        assert loads in (jobs + 1, 2 * jobs + 1), (loads, jobs)
        assert waits <= {0, jobs, jobs + 1}, (jobs, sorted(waits))


@pytest.mark.parametrize("g,tok,odd", INSTANCES)
def test_tile_loop_is_uniform_and_nothing_spills(asm, g, tok, odd):
    lines = kernel(asm, g, tok, odd)
    loop = tile_loop(lines)
    assert not [l for l in loop if re.match(r"s_andn2_b64\s+exec, exec", l)]  # no divergent-loop exit
    assert not [l for l in loop if l.startswith("v_readfirstlane")]
    assert not [l for l in lines if l.startswith("scratch_")]
