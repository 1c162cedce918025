"""Shared pytest setup: import paths and the ``gpu`` marker.

``-m gpu`` tests need an MI355X (gfx950) and the built HIP library; the
``-m "not gpu"`` suite runs on any CPU host.
"""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "composed-mixture-of-experts-engine_amd")
for _p in (PKG_DIR, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
    config.addinivalue_line("markers", "cpu: runs on the CPU only")
