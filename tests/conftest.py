"""Shared test setup.

Markers: ``gpu`` tests need an MI355X and call the HIP library through its C
ABI; everything else runs on the CPU (oracle, host contracts, ABI exports).
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def known_answers():
    return json.loads((GOLDEN / "known_answers.json").read_text())


@pytest.fixture(scope="session")
def native():
    """The built HIP library (tests never build it themselves)."""
    from colormlm_amd import _native

    return _native.lib()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o
