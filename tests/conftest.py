"""pytest configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs on a machine without a GPU (oracle, host logic, C ABI
exports); `-m gpu` runs the kernel parity tests on an MI355X.
"""
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "mlx-recurrence_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
