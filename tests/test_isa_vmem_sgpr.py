"""Every HIP source, compiled for gfx950: no vector-memory instruction reads
an SGPR that a VALU instruction wrote fewer than 5 wait states earlier (see
isa_hazards.vmem_sgpr_hazards).  The kernels issue some loads as inline
assembly, which the compiler does not pad; a descriptor restored with
v_readfirstlane right before such a load would address the wrong memory.
Compiles every source once (about a minute); runs without a GPU."""
import shutil
import subprocess
from pathlib import Path

import pytest

from isa_hazards import vmem_sgpr_hazards
from iris_kernel import _build


@pytest.fixture(scope="module")
def asm_by_source(tmp_path_factory):
    try:
        hipcc = _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if shutil.which(hipcc) is None and not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out_dir = tmp_path_factory.mktemp("isa_sgpr")
    result = {}
    for src, extra in _build.SOURCES.items():
        out = out_dir / (Path(src).stem + ".s")
        cmd = [hipcc, *_build._common_flags(), *extra, "--cuda-device-only", "-S", str(_build.CSRC / src),
               "-o", str(out)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr[-2000:]
        result[src] = out.read_text()
    return result


def test_no_vmem_reads_an_sgpr_right_after_a_valu_write(asm_by_source):
    for src, asm in asm_by_source.items():
        bad = vmem_sgpr_hazards(asm.split("\n"))
        assert not bad, f"{src}: {bad[:5]}"


def test_checker_flags_a_descriptor_restored_by_readfirstlane():
    bad = ["v_readfirstlane_b32 s4, v24",
           "v_readfirstlane_b32 s5, v25",
           "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"]
    load = "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"
    assert vmem_sgpr_hazards(bad) == [(load, 1), (load, 0)]  # s4 one wait state back, s5 none
    padded = ["v_readfirstlane_b32 s4, v24",
              "s_nop 4",
              "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"]
    assert vmem_sgpr_hazards(padded) == []
    salu = ["s_mov_b32 s4, 0", "buffer_load_dwordx4 v[18:21], v29, s[4:7], 0 offen nt"]
    assert vmem_sgpr_hazards(salu) == []
