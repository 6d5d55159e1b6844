import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "iris-kernel_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def asm_by_source(tmp_path_factory):
    """gfx950 assembly of every HIP source of the library, built with the
    library's own flags (no GPU needed; about a minute)."""
    from iris_kernel import _build

    try:
        hipcc = _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if shutil.which(hipcc) is None and not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out_dir = tmp_path_factory.mktemp("isa")
    result = {}
    for src, extra in _build.SOURCES.items():
        out = out_dir / (Path(src).stem + ".s")
        cmd = [hipcc, *_build._common_flags(), *extra, "--cuda-device-only", "-S", str(_build.CSRC / src),
               "-o", str(out)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr[-2000:]
        result[src] = out.read_text()
    return result
