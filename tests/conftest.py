"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs on any CPU host (oracle pins, contracts, ABI symbol and
layout checks).  `-m gpu` tests need an MI355X and call the HIP kernels
through the C ABI; they never fall back to another implementation.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "flash-attention-rdna3_amd"), os.path.join(ROOT, "tests")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
