"""Helpers shared by the GPU parity tests.

Inputs are drawn on the CPU from a seeded numpy generator in float64, rounded
to the kernel's input dtype, and the oracle is fed the rounded values, so the
comparison measures only the kernel's arithmetic.  The metric is the
reference's normalised error max|got - want| / (max|want| + 1e-8)
(_chassis.py:196-199); the bar is 1e-5 for fp32 inputs and 2e-2 for bf16/fp16
inputs.
"""
from __future__ import annotations

import numpy as np
import torch

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}

# Regression guard for 16-bit runs, tighter than the bar above: the kernels
# compute in fp32 (MFMA operands split into bf16 hi + lo), so an output kept
# in fp32 (y, final state, dh0, dA) is accurate to ~1e-5, and a gradient
# stored in bf16 / fp16 carries that format's rounding (2^-9 ~ 2e-3 relative)
# and little else.  A wrong term that stays inside the 2e-2 bar still trips
# these.
GUARD_FP32_OUT = 1e-4
GUARD_16BIT_OUT = 8e-3


def dev():
    return torch.device("cuda:0")


def to_dev(arr, dtype, requires_grad=False):
    t = torch.tensor(np.asarray(arr), dtype=torch.float64).to(dtype).to(dev())
    return t.requires_grad_(requires_grad)


def rounded(t: torch.Tensor) -> np.ndarray:
    """The float64 values the kernel actually sees."""
    return t.detach().to(torch.float64).cpu().numpy()


def rel_err(got, want) -> float:
    got = got.detach().to(torch.float64).cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    want = np.asarray(want, dtype=np.float64)
    return float(np.abs(got - want).max() / (np.abs(want).max() + 1e-8))


def check(name, got, want, tol, report):
    err = rel_err(got, want)
    report[name] = err
    assert np.isfinite(err) and err < tol, f"{name}: normalised error {err:.3e} >= {tol:.1e} ({report})"
    if tol > TOL[torch.float32] and isinstance(got, torch.Tensor):
        guard = GUARD_FP32_OUT if got.dtype == torch.float32 else GUARD_16BIT_OUT
        assert err < guard, f"{name}: normalised error {err:.3e} >= guard {guard:.1e} ({report})"
