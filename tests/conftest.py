"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs the CPU suite (oracle vs the reference's golden vectors,
planner, C-ABI exports); `-m gpu` runs the HIP kernels against the oracle on a
real MI355X.
"""
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "t4a-cuda-kernels_amd", REPO / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP kernels launched)")
