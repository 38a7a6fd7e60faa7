"""Shared fixtures. Tests marked `gpu` need an MI355X (they call the HIP
library through its C ABI); everything else runs on the CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle

    if not oracle.ORACLE_SO.exists():
        oracle.build()
    return oracle.Oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference's own compiled kernels, where oracle/_ref was built."""
    import oracle

    if not oracle.reference_available():
        pytest.skip("oracle/_ref/libnnc_ref.so is not built (the reference sources were absent at build time)")
    return oracle.Reference()
