"""Test configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs the oracle's pinning checks, the host logic and the C-ABI's load/export/validation checks on any
machine; `-m gpu` runs the parity tests of the HIP kernels against the oracle on an MI355X.
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "mako-video_amd", REPO / "oracle", REPO / "tests", REPO / "tests" / "golden"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a GPU")
    return torch.device("cuda:0")
