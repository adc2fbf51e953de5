"""Shared test configuration.

Puts the repository root (for ``oracle``) and ``gfx1010-kernels_amd`` (for the
``gfx1010_kernels`` package) on ``sys.path`` and registers the ``gpu`` marker.
"""

import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
for path in (REPO, REPO / "gfx1010-kernels_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
