import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "kaggle-mltest_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def gemm_asm(tmp_path_factory):
    """nf4_gemm.hip compiled for gfx950 to assembly, once per session (hipcc cross-compiles
    without a GPU): the text, read by the tests of register counts and wait placement."""
    import subprocess

    import build

    try:
        hipcc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "nf4_gemm.s"
    cmd = [hipcc, *build.FLAGS, "--offload-device-only", "-S", str(PKG / "csrc" / "nf4_gemm.hip"),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def pytest_collection_modifyitems(config, items):
    # GPU tests print their case before running, so a GPU fault names it.
    os.environ.setdefault("PYTHONUNBUFFERED", "1")
