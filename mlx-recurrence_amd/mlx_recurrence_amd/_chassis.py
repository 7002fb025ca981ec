"""_chassis.py — shared infrastructure of the scan plug-ins (torch/ROCm host side).

Mirrors ``mlx_recurrence/_chassis.py`` of the reference: the segment-length
default, the lane-width rule, the shape validation with the same conditions
and messages, and the forward+gradient parity helper.  The segment-checkpoint
+ recompute machinery itself lives in the HIP kernels (csrc/*.hip): the
forward writes the state only at chunk boundaries, the backward recomputes
each chunk from its checkpoint and runs the reverse adjoint sweep.

``get_or_build_kernel`` (reference _chassis.py:65-85) JIT-compiles Metal source
strings; this build compiles its kernels ahead of time for gfx950, so the name
is kept only to fail with an explanation.
"""
from __future__ import annotations

import torch

# Default segment length of the checkpoint + recompute pattern
# (reference _chassis.py:51).
DEFAULT_SEG = 32

# Lane-width rule kept from the reference (_chassis.py:55): the lane dimension
# (Dh for SSD/GLA, D for RG-LRU/rotLRU) must be a multiple of 32.
SIMD_WIDTH = 32


def get_or_build_kernel(name, input_names=None, output_names=None, source=None, header=""):
    """Not available: kernels are compiled ahead of time for gfx950.

    The reference compiles Metal source strings at run time
    (_chassis.py:65-85).  Here every kernel is a HIP kernel inside
    librecurrence_gfx950.so, reached through the C ABI in include/recurrence.h.
    """
    raise NotImplementedError(
        "get_or_build_kernel compiles Metal source in mlx-recurrence; the MI355X "
        "kernels are built ahead of time (mlx-recurrence_amd/build.py) and called "
        "through librecurrence_gfx950.so"
    )


def check_segment_shape(L, seg, lane_dim, lane_name="lane dimension"):
    """Validate the segment-checkpoint constraints (reference _chassis.py:92-115).

    Raises:
        ValueError: seg <= 0, L % seg != 0, or lane_dim % 32 != 0, with the
        reference's messages.
    """
    if seg <= 0:
        raise ValueError(f"seg must be positive, got {seg}")
    if L % seg != 0:
        raise ValueError(
            f"sequence length L={L} must be divisible by seg={seg} "
            f"(segment-checkpoint pattern tiles L into L/seg segments)"
        )
    if lane_dim % SIMD_WIDTH != 0:
        raise ValueError(
            f"{lane_name}={lane_dim} must be a multiple of {SIMD_WIDTH} "
            f"(fused gradient reductions use {SIMD_WIDTH}-lane simdgroups)"
        )


def parity_check(
    kernel_fn,
    reference_fn,
    inputs,
    arg_names,
    grad_argnums,
    *,
    w_out=None,
    y_tol=1e-3,
    grad_rtol=1e-3,
    label="",
    verbose=True,
):
    """Compare a kernel against a reference: forward output and every gradient.

    Same protocol as the reference helper (_chassis.py:122-213): the loss is
    ``sum(y * w_out)`` with ``w_out`` drawn from a generator seeded with 1234;
    the forward passes if ``max|y_k - y_r| < y_tol``; each gradient passes if
    ``max|g_k - g_r| / (max|g_r| + 1e-8) < grad_rtol``.

    Returns ``(ok, report)`` with ``report[name] = {"abs": ..., "rel": ...}``.
    """
    inputs = [t.detach().clone().requires_grad_(i in grad_argnums) for i, t in enumerate(inputs)]

    y_k = kernel_fn(*inputs)
    y_r = reference_fn(*inputs)

    if w_out is None:
        gen = torch.Generator().manual_seed(1234)
        w_out = torch.randn(tuple(y_r.shape), generator=gen).to(device=y_r.device, dtype=y_r.dtype)

    report = {}
    ok = True
    y_abs = float((y_k.detach().to(y_r.dtype) - y_r.detach()).abs().max())
    y_scale = float(y_r.detach().abs().max()) + 1e-8
    report["y"] = {"abs": y_abs, "rel": y_abs / y_scale}
    ok = ok and (y_abs < y_tol)

    wanted = [inputs[i] for i in grad_argnums]
    g_k = torch.autograd.grad((y_k * w_out.to(y_k.dtype)).sum(), wanted, allow_unused=True)
    g_r = torch.autograd.grad((y_r * w_out).sum(), wanted, allow_unused=True)

    for i, gk, gr in zip(grad_argnums, g_k, g_r):
        name = arg_names[i]
        gk = torch.zeros_like(inputs[i]) if gk is None else gk
        gr = torch.zeros_like(inputs[i]) if gr is None else gr
        abs_diff = float((gk.double() - gr.double()).abs().max())
        scale = float(gr.double().abs().max()) + 1e-8
        rel = abs_diff / scale
        report[f"grad_{name}"] = {"abs": abs_diff, "rel": rel}
        ok = ok and (rel < grad_rtol)

    if verbose:
        prefix = f"{label}  " if label else ""
        print(f"{prefix}y          max|diff| = {y_abs:.2e}  (rel {report['y']['rel']:.2e})")
        for i in grad_argnums:
            r = report[f"grad_{arg_names[i]}"]
            print(f"{prefix}grad_{arg_names[i]:<8} max|diff| = {r['abs']:.2e}  (rel {r['rel']:.2e})")
        print(f"{prefix}-> {'PASS' if ok else 'FAIL'}")
    return ok, report
