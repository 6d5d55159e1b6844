"""Build libiris_hip.so, the gfx950 HIP kernels behind the iris_kernel API.

``python -m iris_kernel._build`` (with ``iris-kernel_amd`` on ``sys.path``)
or ``build()`` compiles ``csrc/*.hip`` with hipcc for gfx950 and links
``iris_kernel/libiris_hip.so`` in place, next to this file.  The library
depends only on the HIP runtime (libamdhip64.so.7); no torch C++ ABI is
involved, so it loads into any process whose torch is a ROCm 7 build.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent                      # iris-kernel_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"          # repo-level C ABI headers
BUILD_DIR = ROOT / "_build"
LIB_PATH = PKG_DIR / "libiris_hip.so"
ARCH = "gfx950"

# Per-source flags.  The append kernels (append.hip, kv_fp16.hip) must round
# every fp16/fp32 multiply and add separately (their results are bit-exact
# with the reference), so contraction into FMA is disabled there.
SOURCES = {
    "append.hip": ["-ffp-contract=off"],
    "decode.hip": [],
    "decode_pages.hip": [],
    # the streaming kernel takes its prologue scalars in preloaded SGPRs
    "decode_stream.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=10"],
    "decode_mqa.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
    "decode_any.hip": [],
    "decode_hd.hip": [],
    "decode_fp16.hip": [],
    "decode_fp16_stream.hip": [],
    "kv_fp16.hip": ["-ffp-contract=off"],
    "check.hip": [],
}


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    for cand in ("/opt/rocm/bin/hipcc", "hipcc"):
        if cand == "hipcc" or Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Never emit packed fp32 ops (v_pk_fma_f32 & co).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link libiris_hip.so (always rebuilds)."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    for src, extra in SOURCES.items():
        obj = BUILD_DIR / (Path(src).stem + ".o")
        _run([hipcc, *_common_flags(), *extra, "-c", str(CSRC / src), "-o", str(obj)], verbose)
        objs.append(str(obj))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
