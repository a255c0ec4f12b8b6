"""Shared pytest setup: paths, the ``gpu`` marker and per-test banners."""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "piper-offload_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(autouse=True)
def _banner(request: pytest.FixtureRequest) -> None:
    # Name each GPU case on stderr before it runs, so a GPU fault that ends the
    # process still identifies the case that was running.
    if request.node.get_closest_marker("gpu") is not None:
        sys.stderr.write(f"\n[gpu-case] {request.node.nodeid}\n")
        sys.stderr.flush()
