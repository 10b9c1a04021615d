"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs the CPU suite (oracle pins, host logic, ABI surface); `-m gpu` runs the parity
tests, which call the HIP kernels through the C-ABI and compare with the CPU oracle.
"""

import sys

from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent

for path in (ROOT, ROOT / "sonic-sampler_amd", ROOT / "tests"):

    if str(path) not in sys.path:

        sys.path.insert(0, str(path))


def pytest_configure(config):

    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
