"""Shared test configuration.

``-m "not gpu"``: the oracle against the golden vectors, host logic and the
C-ABI library's exports (no GPU work).  ``-m gpu``: parity of the HIP path
against the oracle, run on an MI355X.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    with np.load(ROOT / "tests" / "golden" / "codec_golden.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}
