"""Shared test setup: import paths and the `gpu` marker.

`-m "not gpu"` tests run on any host (oracle vs golden vectors, host logic,
ABI exports).  `-m gpu` tests need an MI355X and call the HIP library
through its C ABI.
"""
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "pytorch-rs_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
