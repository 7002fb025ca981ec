"""mlx_recurrence_amd — fused linear-recurrence scans for AMD MI355X (gfx950).

Drop-in counterpart of the v2 scan API of D-CSIL/mlx-recurrence 0.3.0
(reference mlx_recurrence/__init__.py:22-49) for PyTorch-ROCm tensors:

    ssd     — Mamba-2-style head-wise SSD selective scan
    gla     — Gated Linear Attention recurrence
    rglru   — RG-LRU diagonal recurrence
    rotlru  — rotational LRU (complex-diagonal scan over (u, w) pairs)

Each scan keeps the reference's signature, shape rules and fp32 state /
accumulation, and is differentiable through ``torch.autograd``.  The compute
runs in hand-written HIP kernels for gfx950 (librecurrence_gfx950.so, C ABI in
include/recurrence.h); the ``*_scan_reference`` functions are the per-step
torch loops of the reference for parity testing.

Not carried over: the v0.1 ``legacy`` kernels and their top-level re-exports,
and JIT compilation of kernel source (``get_or_build_kernel`` raises).
"""

from .ssd import ssd_scan, ssd_scan_with_state, ssd_scan_reference
from .gla import gla_scan, gla_scan_with_state, gla_scan_reference
from .rglru import (rglru_scan, rglru_scan_with_state, rglru_scan_reference, rglru_gated_scan,
                    rglru_gated_scan_with_state, rglru_gated_reference)
from .rotlru import (rotlru_scan, rotlru_scan_with_state, rotlru_scan_reference, rotlru_theta_scan,
                     rotlru_theta_scan_with_state)
from ._chassis import DEFAULT_SEG, SIMD_WIDTH, get_or_build_kernel, check_segment_shape, parity_check
from ._lib import async_status
from .step import ssd_step, gla_step, rglru_step, rotlru_step
from .gdn import gated_deltanet_scan, gated_deltanet_scan_with_state, gated_deltanet_reference

__all__ = [
    "ssd_scan",
    "ssd_scan_with_state",
    "ssd_scan_reference",
    "gla_scan",
    "gla_scan_with_state",
    "gla_scan_reference",
    "rglru_scan",
    "rglru_scan_with_state",
    "rglru_scan_reference",
    "rglru_gated_scan",
    "rglru_gated_scan_with_state",
    "rglru_gated_reference",
    "rotlru_scan",
    "rotlru_scan_with_state",
    "rotlru_scan_reference",
    "rotlru_theta_scan",
    "rotlru_theta_scan_with_state",
    "DEFAULT_SEG",
    "SIMD_WIDTH",
    "get_or_build_kernel",
    "check_segment_shape",
    "parity_check",
    "async_status",
    "ssd_step",
    "gla_step",
    "rglru_step",
    "rotlru_step",
    "gated_deltanet_scan",
    "gated_deltanet_scan_with_state",
    "gated_deltanet_reference",
]

__version__ = "0.3.0+gfx950"
