"""Test configuration: import paths, the ``gpu`` marker, and one-time builds.

``-m "not gpu"`` runs everything that needs no GPU: the format, the codec,
the oracle against the reference's vectors, and the C ABI's host-side
contract.  ``-m gpu`` runs the parity tests of the HIP kernels through the
C ABI on a real MI355X.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "mlx-iqk_amd", ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: exhaustive sweeps")
    _ensure_built()


def _ensure_built() -> None:
    """Build what is missing (never rebuild what exists: build() does that)."""
    from mlx_iqk_amd import build
    if not build.CODEC_LIB.is_file():
        build.build_codec()
    from oracle import oracle
    if not oracle.ORACLE_LIB.is_file() or (oracle.REFERENCE_SOURCES.is_dir() and not oracle.ref_available()):
        oracle.build()


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("this test needs a GPU (run with -m 'not gpu' on a CPU-only host)")
    from mlx_iqk_amd import _native
    _native.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")
