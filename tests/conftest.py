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


import pytest  # noqa: E402


@pytest.fixture(autouse=True)
def _kernel_status_after_gpu_tests(request):
    """After every GPU test: synchronise and fail the test if a kernel reported
    an error after its launch returned (rr_async_status, e.g. an expired tile
    hand-off wait whose results were NaN-marked)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import torch
    if not torch.cuda.is_available():
        return
    from mlx_recurrence_amd import _lib
    _lib.async_status()
