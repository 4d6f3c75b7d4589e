"""Test lanes: the default lane runs on the CPU (oracle, golden fixtures, planner, C-ABI exports,
API validation); `-m gpu` tests need an MI355X and call the HIP kernels through the C-ABI."""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "mlx-train-perf_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP extension")
