"""pytest configuration: the `gpu` marker and in-tree imports.

GPU tests need a real MI355X (run with ``-m gpu``); everything else runs on
the CPU.  Tests load the in-tree libraries and build them only when none is
present.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    from strataflow_amd import build
    if not build.LIB.exists():
        build.build_hip()
    if not build.HOST_LIB.exists():
        build.build_host()
    if not (build.ORACLE_DIR / "liboracle.so").exists():
        build.build_oracle()


_ensure_built()


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle
    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test needs a GPU (run with -m 'not gpu' on CPU-only hosts)")
    return torch.device("cuda:0")
