"""pytest setup: import paths and the `gpu` marker.

`-m "not gpu"` runs the CPU suite (oracle pins, golden vectors, host logic,
the C-ABI library's exports); `-m gpu` runs the parity tests that call the
HIP kernels through the C ABI on an MI355X.
"""

from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "hetero-serve_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libhsattn.so")
