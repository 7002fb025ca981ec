"""rotlru.py — rotational LRU: pair-diagonal complex scan over interleaved (u, w).

Host side of the rotLRU plug-in (reference mlx_recurrence/rotlru.py)::

    [u]       [c_t  -s_t] [u]         [x_t[2p]  ]
    [w]  = a_t[s_t   c_t] [w]      +  [x_t[2p+1]]
       t                     t-1

``cs``/``sn`` are supplied by the caller (cos/sin of an angle computed in torch,
so angle gradients chain through autograd, rotlru.py:18-23).  The kernel is
range-agnostic: ``a`` may be negative and (cs, sn) need not be normalised.

Public API (reference rotlru.py:297-351):
    rotlru_scan(a, cs, sn, x, seg=32)              -> y  [B, L, 2*Dp] fp32
    rotlru_scan_with_state(a, cs, sn, x, seg=32)   -> (y, final_state [B, 2*Dp])
    rotlru_scan_reference(a, cs, sn, x)            -> y  (per-step torch loop)

Beyond the reference: keyword-only ``initial_state`` [B, 2*Dp] and the
gradient of a loss that uses ``final_state`` (dropped by the reference VJP,
rotlru.py:289).
"""
from __future__ import annotations

import torch

from . import _lib
from ._chassis import DEFAULT_SEG, check_segment_shape


def _validate(a, cs, sn, x):
    """Shape rules and messages of the reference _validate (rotlru.py:61-73)."""
    if a.ndim != 3:
        raise ValueError(f"a must be [B, L, Dp], got shape {tuple(a.shape)}")
    if tuple(a.shape) != tuple(cs.shape) or tuple(a.shape) != tuple(sn.shape):
        raise ValueError(
            f"a/cs/sn shapes must match, got {tuple(a.shape)}, {tuple(cs.shape)}, {tuple(sn.shape)}"
        )
    B, L, Dp = a.shape
    if tuple(x.shape) != (B, L, 2 * Dp):
        raise ValueError(f"x must be [B, L, 2*Dp] = [{B}, {L}, {2 * Dp}], got {tuple(x.shape)}")
    return B, L, Dp


class _RotLRUScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, cs, sn, x, h0, seg):
        dev = _lib.require_device(a, cs, sn, x, h0)
        dt = _lib.common_dtype(a, cs, sn, x)
        a_, cs_, sn_, x_ = (_lib.prep(t, dt) for t in (a, cs, sn, x))
        B, L, Dp = a_.shape
        D = 2 * Dp
        h0_ = None if h0 is None else _lib.prep(h0.reshape(B, D), torch.float32)
        nC = L // _lib.chunk_len(L, seg)
        y = torch.empty((B, L, D), dtype=torch.float32, device=dev)
        ckpt = torch.empty((B, nC, D), dtype=torch.float32, device=dev)
        with _lib.device_guard(dev):
            ws = _lib.rotlru_workspace(B, L, Dp, seg, dt, 0, dev)
            _lib.rotlru_fwd(a_, cs_, sn_, x_, h0_, seg, y, ckpt, ws)
        ctx.save_for_backward(a_, cs_, sn_, x_, h0_, ckpt)
        ctx.seg = seg
        ctx.set_materialize_grads(False)
        return y, ckpt[:, -1]

    @staticmethod
    def backward(ctx, dy, dfinal):
        a_, cs_, sn_, x_, h0_, ckpt = ctx.saved_tensors
        B, L, Dp = a_.shape
        D = 2 * Dp
        dev = a_.device
        dy = torch.zeros((B, L, D), dtype=torch.float32, device=dev) if dy is None else _lib.prep(dy, torch.float32)
        dfinal = None if dfinal is None else _lib.prep(dfinal, torch.float32)
        da, dcs, dsn = torch.empty_like(a_), torch.empty_like(cs_), torch.empty_like(sn_)
        dx = torch.empty_like(x_)
        dh0 = torch.empty((B, D), dtype=torch.float32, device=dev) if ctx.needs_input_grad[4] else None
        with _lib.device_guard(dev):
            ws = _lib.rotlru_workspace(B, L, Dp, ctx.seg, a_.dtype, 1, dev)
            _lib.rotlru_bwd(dy, dfinal, a_, cs_, sn_, x_, h0_, ckpt, ctx.seg, da, dcs, dsn, dx, dh0, ws)
        return da, dcs, dsn, dx, dh0, None


def _run(a, cs, sn, x, seg, initial_state):
    B, L, Dp = _validate(a, cs, sn, x)
    check_segment_shape(L, seg, x.shape[2], "D")
    if initial_state is not None and tuple(initial_state.shape) != (B, 2 * Dp):
        raise ValueError(f"initial_state must be [B, 2*Dp] = [{B}, {2 * Dp}], got {tuple(initial_state.shape)}")
    return _RotLRUScan.apply(a, cs, sn, x, initial_state, seg)


def rotlru_scan(a, cs, sn, x, seg=DEFAULT_SEG, *, initial_state=None):
    """Rotational LRU pair-diagonal scan on the GPU (fused forward + backward).

    Args:
        a:   [B, L, Dp] per-pair magnitude gate (any real value).
        cs:  [B, L, Dp] cos(theta_t).
        sn:  [B, L, Dp] sin(theta_t).
        x:   [B, L, D] drive, D = 2*Dp, pairs interleaved (u, w).
        seg: checkpoint segment length (L % seg == 0; default 32).

    Returns:
        y:   [B, L, D] float32, interleaved like x.

    ``D`` must be a multiple of 32.
    """
    y, _ = _run(a, cs, sn, x, seg, initial_state)
    return y


def rotlru_scan_with_state(a, cs, sn, x, seg=DEFAULT_SEG, *, initial_state=None):
    """Rotational LRU scan that also returns the final state [B, D] (interleaved)."""
    return _run(a, cs, sn, x, seg, initial_state)


def rotlru_scan_reference(a, cs, sn, x, *, initial_state=None):
    """Per-step torch loop, op for op as the reference's rotlru_scan_reference
    (rotlru.py:338-351).  Differentiable; runs on any device."""
    B, L, Dp = _validate(a, cs, sn, x)
    ct = torch.float32
    for t in (a, cs, sn, x):
        ct = torch.promote_types(ct, t.dtype)
    xp = x.to(ct).reshape(B, L, Dp, 2)
    if initial_state is None:
        u = torch.zeros((B, Dp), dtype=ct, device=a.device)
        w = torch.zeros((B, Dp), dtype=ct, device=a.device)
    else:
        h0 = initial_state.to(ct).reshape(B, Dp, 2)
        u, w = h0[..., 0], h0[..., 1]
    ys = []
    # per-step slices from unbind (one backward stack, not a scatter per step)
    for at, c, s, x_t in zip(a.to(ct).unbind(1), cs.to(ct).unbind(1), sn.to(ct).unbind(1), xp.unbind(1)):
        un = at * (c * u - s * w) + x_t[:, :, 0]
        wn = at * (s * u + c * w) + x_t[:, :, 1]
        u, w = un, wn
        ys.append(torch.stack([u, w], dim=-1).reshape(B, 2 * Dp))
    return torch.stack(ys, dim=1)


# ------------------------------------------------------ rotLRU from theta
class _RotLRUThetaScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, th, x, h0, seg):
        dev = _lib.require_device(a, th, x, h0)
        dt = _lib.common_dtype(a, th, x)
        a_, th_, x_ = (_lib.prep(t, dt) for t in (a, th, x))
        B, L, Dp = a_.shape
        D = 2 * Dp
        h0_ = None if h0 is None else _lib.prep(h0.reshape(B, D), torch.float32)
        nC = L // _lib.chunk_len(L, seg)
        y = torch.empty((B, L, D), dtype=torch.float32, device=dev)
        ckpt = torch.empty((B, nC, D), dtype=torch.float32, device=dev)
        with _lib.device_guard(dev):
            ws = _lib.rotlru_workspace(B, L, Dp, seg, dt, 0, dev)
            _lib.rotlru_theta_fwd(a_, th_, x_, h0_, seg, y, ckpt, ws)
        ctx.save_for_backward(a_, th_, x_, h0_, ckpt)
        ctx.seg = seg
        ctx.set_materialize_grads(False)
        return y, ckpt[:, -1]

    @staticmethod
    def backward(ctx, dy, dfinal):
        a_, th_, x_, h0_, ckpt = ctx.saved_tensors
        B, L, Dp = a_.shape
        D = 2 * Dp
        dev = a_.device
        dy = torch.zeros((B, L, D), dtype=torch.float32, device=dev) if dy is None else _lib.prep(dy, torch.float32)
        dfinal = None if dfinal is None else _lib.prep(dfinal, torch.float32)
        da, dth, dx = torch.empty_like(a_), torch.empty_like(th_), torch.empty_like(x_)
        dh0 = torch.empty((B, D), dtype=torch.float32, device=dev) if ctx.needs_input_grad[3] else None
        with _lib.device_guard(dev):
            ws = _lib.rotlru_workspace(B, L, Dp, ctx.seg, a_.dtype, 1, dev)
            _lib.rotlru_theta_bwd(dy, dfinal, a_, th_, x_, h0_, ckpt, ctx.seg, da, dth, dx, dh0, ws)
        return da, dth, dx, dh0, None


def _run_theta(a, theta, x, seg, initial_state):
    B, L, Dp = _validate(a, theta, theta, x)
    check_segment_shape(L, seg, 2 * Dp, "D")
    if initial_state is not None and tuple(initial_state.shape) != (B, 2 * Dp):
        raise ValueError(f"initial_state must be [B, 2*Dp] = [{B}, {2 * Dp}], got {tuple(initial_state.shape)}")
    return _RotLRUThetaScan.apply(a, theta, x, initial_state, seg)


def rotlru_theta_scan(a, theta, x, seg=DEFAULT_SEG, *, initial_state=None):
    """rotlru_scan with the rotation given by its angle: the kernels form
    cos(theta) and sin(theta) in registers (the reference forms them in MLX
    host code, rotlru.py:18-23) and return d theta = -sin * dcs + cos * dsn.
    a, theta [B, L, Dp]; x [B, L, 2*Dp] interleaved (u, w) pairs."""
    y, _ = _run_theta(a, theta, x, seg, initial_state)
    return y


def rotlru_theta_scan_with_state(a, theta, x, seg=DEFAULT_SEG, *, initial_state=None):
    """rotlru_theta_scan that also returns the final state [B, 2*Dp]."""
    return _run_theta(a, theta, x, seg, initial_state)
