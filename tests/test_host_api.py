"""Host-side API behaviour that needs no GPU: the shape rules raise ValueError
with the reference's messages before any device work, CPU tensors are refused
(no CPU fallback), and the chassis mirrors the reference."""
import pytest
import torch

import mlx_recurrence_amd as mr
from mlx_recurrence_amd import _chassis


def test_public_names_match_reference_v2_api():
    # reference mlx_recurrence/__init__.py:60-88 minus the legacy re-exports
    for name in ["ssd_scan", "ssd_scan_with_state", "ssd_scan_reference", "gla_scan",
                 "gla_scan_with_state", "gla_scan_reference", "rglru_scan",
                 "rglru_scan_with_state", "rglru_scan_reference", "rotlru_scan",
                 "rotlru_scan_with_state", "rotlru_scan_reference", "DEFAULT_SEG",
                 "get_or_build_kernel", "check_segment_shape", "parity_check"]:
        assert hasattr(mr, name), name
    assert mr.DEFAULT_SEG == 32


def test_check_segment_shape_messages():
    with pytest.raises(ValueError, match="seg must be positive, got 0"):
        _chassis.check_segment_shape(64, 0, 32)
    with pytest.raises(ValueError, match=r"sequence length L=30 must be divisible by seg=32"):
        _chassis.check_segment_shape(30, 32, 32)
    with pytest.raises(ValueError, match=r"Dh=16 must be a multiple of 32"):
        _chassis.check_segment_shape(32, 32, 16, "Dh")
    _chassis.check_segment_shape(96, 16, 32, "Dh")


def test_get_or_build_kernel_explains():
    with pytest.raises(NotImplementedError):
        mr.get_or_build_kernel("x", [], [], "")


def _ssd(B, L, H, Dh, N):
    return (torch.randn(B, L, H, Dh), torch.rand(B, L, H), torch.randn(B, L, H, N),
            torch.randn(B, L, H, N), -torch.rand(H, N) - 0.1)


def test_invalid_shapes_raise_value_error():
    # test_v2_ssd.py:63-72, test_v2_gla.py:56-63, test_v2_rglru.py:54-61, test_v2_rotlru.py:126-135
    with pytest.raises(ValueError):
        mr.ssd_scan(*_ssd(1, 30, 2, 32, 8), seg=32)
    with pytest.raises(ValueError):
        mr.ssd_scan(*_ssd(1, 32, 2, 16, 8), seg=32)
    q = torch.randn(1, 30, 2, 32)
    with pytest.raises(ValueError):
        mr.gla_scan(q, q, q, torch.rand(1, 30, 2), seg=32)
    q = torch.randn(1, 32, 2, 16)
    with pytest.raises(ValueError):
        mr.gla_scan(q, q, q, torch.rand(1, 32, 2), seg=32)
    with pytest.raises(ValueError):
        mr.rglru_scan(torch.rand(1, 30, 32), torch.rand(1, 30, 32), seg=32)
    with pytest.raises(ValueError):
        mr.rglru_scan(torch.rand(1, 32, 16), torch.rand(1, 32, 16), seg=32)
    a = torch.rand(1, 48, 16)
    with pytest.raises(ValueError):
        mr.rotlru_scan(a, a, a, torch.rand(1, 48, 32))
    a = torch.rand(1, 64, 8)
    with pytest.raises(ValueError):
        mr.rotlru_scan(a, a, a, torch.rand(1, 64, 16))
    a = torch.rand(1, 64, 16)
    with pytest.raises(ValueError, match=r"x must be \[B, L, 2\*Dp\]"):
        mr.rotlru_scan(a, a, a, torch.rand(1, 64, 30))
    with pytest.raises(ValueError, match="a/cs/sn shapes must match"):
        mr.rotlru_scan(a, a[:, :, :8], a, torch.rand(1, 64, 32))
    with pytest.raises(ValueError, match="A_neg must be"):
        u, d, B, C, _ = _ssd(1, 32, 2, 32, 8)
        mr.ssd_scan(u, d, B, C, -torch.rand(3))        # H = 2
    with pytest.raises(ValueError, match="A_neg must be"):
        mr.ssd_scan(u, d, B, C, -torch.rand(2, 8, 1))


def test_cpu_tensors_are_refused():
    """The product path has no CPU fallback."""
    a = torch.rand(1, 32, 32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mr.rglru_scan(a, a)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mr.ssd_scan(*_ssd(1, 32, 2, 32, 8))


def test_parity_check_reference_vs_itself():
    """parity_check's protocol on CPU with the reference loop on both sides."""
    torch.manual_seed(0)
    a = torch.sigmoid(torch.randn(2, 16, 8) + 2)
    x = torch.randn(2, 16, 8)
    ok, rep = mr.parity_check(mr.rglru_scan_reference, mr.rglru_scan_reference, (a, x),
                              ["a", "x"], (0, 1), verbose=False)
    assert ok and rep["y"]["abs"] == 0.0 and rep["grad_a"]["rel"] == 0.0


def test_ssd_reference_takes_per_head_rates():
    """A 1-D A_neg [H] is one rate per head: the reference loop gives the same
    y as with A[:, None].expand(H, N), and its gradient is the per-head sum."""
    u, d, B, C, _ = _ssd(2, 16, 3, 32, 8)
    A = -torch.rand(3, dtype=torch.float64) - 0.1
    A1 = A.clone().requires_grad_(True)
    A2 = A.clone().requires_grad_(True)
    y1 = mr.ssd_scan_reference(u.double(), d.double(), B.double(), C.double(), A1)
    y2 = mr.ssd_scan_reference(u.double(), d.double(), B.double(), C.double(), A2[:, None].expand(3, 8))
    assert torch.equal(y1, y2)
    w = torch.randn_like(y1)
    (y1 * w).sum().backward()
    (y2 * w).sum().backward()
    torch.testing.assert_close(A1.grad, A2.grad, rtol=1e-12, atol=1e-12)
