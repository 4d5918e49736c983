"""Shared pytest configuration.

Markers: ``gpu`` tests need an MI355X (gfx950) and the built HIP library;
everything else runs on the CPU.  ``tests/`` may import the CPU oracle under
``oracle/``; product code never does.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as module

    module.build()
    return module
