"""pytest configuration: import paths and the ``gpu`` marker.

``gpu`` marks tests that need a HIP device (the reference's convention, pyproject.toml:38-41).
"""

from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for path in (ROOT / "moss-image_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires a HIP device (MI355X)")
