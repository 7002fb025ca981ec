"""rglru.py — RG-LRU diagonal scan ``h_t = a_t * h_{t-1} + x_t`` (y_t = h_t).

Host side of the RG-LRU plug-in (reference mlx_recurrence/rglru.py).  The gate
math of RG-LRU (``a_t = exp(-c softplus(Lambda) sigmoid(r_t))``,
``x_t = sqrt(1 - a_t^2) (i_t x_t)``) stays in ordinary torch code, as in the
reference (rglru.py:19-27); the kernel is the sequential scan.

Public API (reference rglru.py:234-282):
    rglru_scan(a, x, seg=32)               -> y        [B, L, D] fp32
    rglru_scan_with_state(a, x, seg=32)    -> (y, final_state [B, D])
    rglru_scan_reference(a, x)             -> y        (per-step torch loop)

Beyond the reference: a keyword-only ``initial_state`` [B, D] (chunked
prefill / continuation), the gradient of a loss that uses ``final_state``
(the reference VJP drops that cotangent, rglru.py:226), and
``rglru_gated_scan(r, i, x, lam, c)``, which fuses the gate math into the
scan kernels so that a and x' never travel through HBM.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._chassis import DEFAULT_SEG, check_segment_shape


def _validate(a, x):
    if a.ndim != 3:
        raise ValueError(f"a must be [B, L, D], got shape {tuple(a.shape)}")
    if tuple(x.shape) != tuple(a.shape):
        raise ValueError(f"a and x shapes must match, got {tuple(a.shape)} and {tuple(x.shape)}")
    return a.shape


class _RGLRUScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, x, h0, seg):
        dev = _lib.require_device(a, x, h0)
        dt = _lib.common_dtype(a, x)
        a_, x_ = _lib.prep(a, dt), _lib.prep(x, dt)
        B, L, D = a_.shape
        h0_ = None if h0 is None else _lib.prep(h0.reshape(B, D), torch.float32)
        nC = L // _lib.chunk_len(L, seg)
        y = torch.empty((B, L, D), dtype=torch.float32, device=dev)
        ckpt = torch.empty((B, nC, D), dtype=torch.float32, device=dev)
        with _lib.device_guard(dev):
            ws = _lib.rglru_workspace(B, L, D, seg, dt, 0, dev)
            _lib.rglru_fwd(a_, x_, h0_, seg, y, ckpt, ws)
        ctx.save_for_backward(a_, x_, h0_, ckpt)
        ctx.seg = seg
        ctx.set_materialize_grads(False)
        return y, ckpt[:, -1]

    @staticmethod
    def backward(ctx, dy, dfinal):
        a_, x_, h0_, ckpt = ctx.saved_tensors
        B, L, D = a_.shape
        dev = a_.device
        dy = torch.zeros((B, L, D), dtype=torch.float32, device=dev) if dy is None else _lib.prep(dy, torch.float32)
        dfinal = None if dfinal is None else _lib.prep(dfinal, torch.float32)
        da = torch.empty_like(a_)
        dx = torch.empty_like(x_)
        dh0 = torch.empty((B, D), dtype=torch.float32, device=dev) if ctx.needs_input_grad[2] else None
        with _lib.device_guard(dev):
            ws = _lib.rglru_workspace(B, L, D, ctx.seg, a_.dtype, 1, dev)
            _lib.rglru_bwd(dy, dfinal, a_, x_, h0_, ckpt, ctx.seg, da, dx, dh0, ws)
        return da, dx, dh0, None


def _run(a, x, seg, initial_state):
    B, L, D = _validate(a, x)
    check_segment_shape(L, seg, D, "D")
    if initial_state is not None and tuple(initial_state.shape) != (B, D):
        raise ValueError(f"initial_state must be [B, D] = [{B}, {D}], got {tuple(initial_state.shape)}")
    return _RGLRUScan.apply(a, x, initial_state, seg)


def rglru_scan(a, x, seg=DEFAULT_SEG, *, initial_state=None):
    """RG-LRU diagonal linear scan on the GPU (fused forward + backward).

    Computes ``h_t = a_t * h_{t-1} + x_t`` and returns ``y_t = h_t`` for all t
    (carry starts at ``initial_state``, zero by default).

    Args:
        a:   [B, L, D] per-channel recurrent gate (any real value).
        x:   [B, L, D] the already-gated input (rglru.py:243-245).
        seg: checkpoint segment length (L % seg == 0; default 32).

    Returns:
        y:   [B, L, D] float32.

    ``D`` must be a multiple of 32.  fp32 state/accumulation; bf16/fp16 inputs
    are widened on load.
    """
    y, _ = _run(a, x, seg, initial_state)
    return y


def rglru_scan_with_state(a, x, seg=DEFAULT_SEG, *, initial_state=None):
    """RG-LRU scan that also returns the final state [B, D] for chunked prefill."""
    return _run(a, x, seg, initial_state)


def rglru_scan_reference(a, x, *, initial_state=None):
    """Per-step torch loop, op for op as the reference's rglru_scan_reference
    (rglru.py:274-282).  Differentiable; runs on any device."""
    B, L, D = a.shape
    ct = torch.promote_types(torch.promote_types(a.dtype, x.dtype), torch.float32)
    h = torch.zeros((B, D), dtype=ct, device=a.device) if initial_state is None else initial_state.to(ct)
    ys = []
    # per-step slices from unbind (one backward stack, not a scatter per step)
    for a_t, x_t in zip(a.to(ct).unbind(1), x.to(ct).unbind(1)):
        h = a_t * h + x_t
        ys.append(h)
    return torch.stack(ys, dim=1)


# ------------------------------------------------------------ gated RG-LRU
class _RGLRUGatedScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, i, x, lam, h0, c, seg):
        dev = _lib.require_device(r, i, x, lam, h0)
        dt = _lib.common_dtype(r, i, x)
        r_, i_, x_ = _lib.prep(r, dt), _lib.prep(i, dt), _lib.prep(x, dt)
        lam_ = _lib.prep(lam, torch.float32)
        B, L, D = r_.shape
        h0_ = None if h0 is None else _lib.prep(h0.reshape(B, D), torch.float32)
        nC = L // _lib.chunk_len(L, seg)
        y = torch.empty((B, L, D), dtype=torch.float32, device=dev)
        ckpt = torch.empty((B, nC, D), dtype=torch.float32, device=dev)
        with _lib.device_guard(dev):
            ws = _lib.rglru_gated_workspace(B, L, D, seg, dt, 0, dev)
            _lib.rglru_gated_fwd(r_, i_, x_, lam_, c, h0_, seg, y, ckpt, ws)
        ctx.save_for_backward(r_, i_, x_, lam_, h0_, ckpt)
        ctx.c, ctx.seg = c, seg
        ctx.set_materialize_grads(False)
        return y, ckpt[:, -1]

    @staticmethod
    def backward(ctx, dy, dfinal):
        r_, i_, x_, lam_, h0_, ckpt = ctx.saved_tensors
        B, L, D = r_.shape
        dev = r_.device
        dy = torch.zeros((B, L, D), dtype=torch.float32, device=dev) if dy is None else _lib.prep(dy, torch.float32)
        dfinal = None if dfinal is None else _lib.prep(dfinal, torch.float32)
        dr, di, dx = (torch.empty_like(t) for t in (r_, i_, x_))
        dlam = torch.empty((D,), dtype=torch.float32, device=dev)
        dh0 = torch.empty((B, D), dtype=torch.float32, device=dev) if ctx.needs_input_grad[4] else None
        with _lib.device_guard(dev):
            ws = _lib.rglru_gated_workspace(B, L, D, ctx.seg, r_.dtype, 1, dev)
            _lib.rglru_gated_bwd(dy, dfinal, r_, i_, x_, lam_, ctx.c, h0_, ckpt, ctx.seg, dr, di, dx, dlam, dh0, ws)
        return dr, di, dx, dlam, dh0, None, None


def _run_gated(r, i, x, lam, c, seg, initial_state):
    B, L, D = _validate(r, x)
    if tuple(i.shape) != (B, L, D):
        raise ValueError(f"i must match r and x, got {tuple(i.shape)}")
    if lam.ndim != 1 or lam.shape[0] != D:
        raise ValueError(f"lam must be [D] = [{D}], got {tuple(lam.shape)}")
    if not (float(c) > 0 and math.isfinite(float(c))):
        raise ValueError(f"c must be positive and finite, got {c}")
    check_segment_shape(L, seg, D, "D")
    if initial_state is not None and tuple(initial_state.shape) != (B, D):
        raise ValueError(f"initial_state must be [B, D] = [{B}, {D}], got {tuple(initial_state.shape)}")
    return _RGLRUGatedScan.apply(r, i, x, lam, initial_state, float(c), seg)


def rglru_gated_scan(r, i, x, lam, c=8.0, seg=DEFAULT_SEG, *, initial_state=None):
    """RG-LRU with its gate math fused into the scan kernels.

    Computes, per channel d (reference rglru.py:10-17, whose gate math runs in
    MLX host code before the scan kernel):
        a_t  = exp(-c * softplus(lam[d]) * sigmoid(r_t))
        h_t  = a_t * h_{t-1} + sqrt(1 - a_t^2) * (i_t * x_t)
    and returns y_t = h_t.  Gradients flow to r, i, x, lam (summed over batch
    and steps) and initial_state.

    Args:
        r:   [B, L, D] recurrence-gate pre-activation.
        i:   [B, L, D] input gate (already activated).
        x:   [B, L, D] input.
        lam: [D] per-channel decay parameter (fp32).
        c:   gate scale (Griffin: 8).
    """
    y, _ = _run_gated(r, i, x, lam, c, seg, initial_state)
    return y


def rglru_gated_scan_with_state(r, i, x, lam, c=8.0, seg=DEFAULT_SEG, *, initial_state=None):
    """rglru_gated_scan that also returns the final state [B, D]."""
    return _run_gated(r, i, x, lam, c, seg, initial_state)


def rglru_gated_reference(r, i, x, lam, c=8.0, *, initial_state=None):
    """The gate math as plain torch ops followed by rglru_scan_reference (the
    composition the reference runs in MLX, rglru.py:13-14 and :274-282)."""
    ct = torch.promote_types(torch.promote_types(r.dtype, x.dtype), torch.float32)
    a = torch.exp(-c * torch.nn.functional.softplus(lam.to(ct)) * torch.sigmoid(r.to(ct)))
    xg = torch.sqrt(1 - a * a) * (i.to(ct) * x.to(ct))
    return rglru_scan_reference(a, xg, initial_state=initial_state)
