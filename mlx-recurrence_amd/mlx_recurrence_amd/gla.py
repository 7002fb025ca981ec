"""gla.py — Gated Linear Attention recurrence (checkpoint + recompute).

Host side of the GLA plug-in (reference mlx_recurrence/gla.py).  Per head the
state is the Dh x Dh matrix S with one scalar forget gate per token::

    S_t[i, j] = g_t * S_{t-1}[i, j] + k_t[i] * v_t[j]
    o_t[j]    = sum_i q_t[i] * S_t[i, j]          (post-update state)

Public API (reference gla.py:301-346):
    gla_scan(q, k, v, gates, seg=32)              -> y [B, L, H, Dh] fp32
    gla_scan_with_state(q, k, v, gates, seg=32)   -> (y, final_state [B, H, Dh, Dh])
    gla_scan_reference(q, k, v, gates)            -> y (per-step torch loop)

Beyond the reference: keyword-only ``initial_state`` [B, H, Dh, Dh] and the
gradient of a loss that uses ``final_state`` (dropped by the reference VJP,
gla.py:293).
"""
from __future__ import annotations

import torch

from . import _lib
from ._chassis import DEFAULT_SEG, check_segment_shape


def _validate(q, k, v, gates):
    if q.ndim != 4:
        raise ValueError(f"q must be [B, L, H, Dh], got shape {tuple(q.shape)}")
    B, L, H, Dh = q.shape
    for name, t in (("k", k), ("v", v)):
        if tuple(t.shape) != (B, L, H, Dh):
            raise ValueError(f"{name} must be [B, L, H, Dh] = [{B}, {L}, {H}, {Dh}], got {tuple(t.shape)}")
    if tuple(gates.shape) != (B, L, H):
        raise ValueError(f"gates must be [B, L, H] = [{B}, {L}, {H}], got {tuple(gates.shape)}")
    return B, L, H, Dh


class _GLAScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gates, h0, seg):
        dev = _lib.require_device(q, k, v, gates, h0)
        dt = _lib.common_dtype(q, k, v, gates)
        q_, k_, v_, g_ = (_lib.prep(t, dt) for t in (q, k, v, gates))
        B, L, H, Dh = q_.shape
        h0_ = None if h0 is None else _lib.prep(h0, torch.float32)
        nC = L // _lib.chunk_len(L, seg)
        y = torch.empty((B, L, H, Dh), dtype=torch.float32, device=dev)
        ckpt = torch.empty((B, H, nC, Dh, Dh), dtype=torch.float32, device=dev)
        with _lib.device_guard(dev):
            ws = _lib.gla_workspace(B, L, H, Dh, seg, dt, 0, dev)
            _lib.gla_fwd(q_, k_, v_, g_, h0_, seg, y, ckpt, ws)
        ctx.save_for_backward(q_, k_, v_, g_, h0_, ckpt)
        ctx.seg = seg
        ctx.set_materialize_grads(False)
        # ckpt stores S[i, j] with i fastest ([.., j, i]); the state is [.., i, j].
        return y, ckpt[:, :, -1].transpose(-1, -2)

    @staticmethod
    def backward(ctx, dy, dfinal):
        q_, k_, v_, g_, h0_, ckpt = ctx.saved_tensors
        B, L, H, Dh = q_.shape
        dev = q_.device
        dy = torch.zeros((B, L, H, Dh), dtype=torch.float32, device=dev) if dy is None else _lib.prep(dy, torch.float32)
        dfinal = None if dfinal is None else _lib.prep(dfinal, torch.float32)
        dq, dk, dv, dg = (torch.empty_like(t) for t in (q_, k_, v_, g_))
        dh0 = torch.empty((B, H, Dh, Dh), dtype=torch.float32, device=dev) if ctx.needs_input_grad[4] else None
        with _lib.device_guard(dev):
            ws = _lib.gla_workspace(B, L, H, Dh, ctx.seg, q_.dtype, 1, dev)
            _lib.gla_bwd(dy, dfinal, q_, k_, v_, g_, h0_, ckpt, ctx.seg, dq, dk, dv, dg, dh0, ws)
        return dq, dk, dv, dg, dh0, None


def _run(q, k, v, gates, seg, initial_state):
    B, L, H, Dh = _validate(q, k, v, gates)
    check_segment_shape(L, seg, Dh, "Dh")
    if initial_state is not None and tuple(initial_state.shape) != (B, H, Dh, Dh):
        raise ValueError(
            f"initial_state must be [B, H, Dh, Dh] = [{B}, {H}, {Dh}, {Dh}], got {tuple(initial_state.shape)}"
        )
    ext = _lib.autograd_ext()
    if ext is not None:   # the same forward / backward as one C++ autograd node
        return ext.gla_scan(q, k, v, gates, initial_state, seg)
    return _GLAScan.apply(q, k, v, gates, initial_state, seg)


def gla_scan(q, k, v, gates, seg=DEFAULT_SEG, *, initial_state=None):
    """Gated Linear Attention recurrence on the GPU (fused forward + backward).

    Args:
        q, k, v: [B, L, H, Dh]  queries (pre-scaled), keys, values
        gates:   [B, L, H]      scalar forget gate per head
        seg:     checkpoint segment length (L % seg == 0; default 32)

    Returns:
        y:       [B, L, H, Dh] float32

    ``Dh`` must be a multiple of 32.  fp32 state/accumulation internally.
    """
    y, _ = _run(q, k, v, gates, seg, initial_state)
    return y


def gla_scan_with_state(q, k, v, gates, seg=DEFAULT_SEG, *, initial_state=None):
    """GLA scan that also returns the final state [B, H, Dh, Dh] (S[i, j])."""
    return _run(q, k, v, gates, seg, initial_state)


def gla_scan_reference(q, k, v, gates, *, initial_state=None):
    """Per-step torch loop, op for op as the reference's gla_scan_reference
    (gla.py:336-346).  Differentiable; runs on any device."""
    B, L, H, Dh = q.shape
    ct = torch.float32
    for t in (q, k, v, gates):
        ct = torch.promote_types(ct, t.dtype)
    q, k, v, gates = (t.to(ct) for t in (q, k, v, gates))
    h = torch.zeros((B, H, Dh, Dh), dtype=ct, device=q.device) if initial_state is None else initial_state.to(ct)
    ys = []
    # per-step slices from unbind (one backward stack, not a scatter per step)
    for g_t, k_t, v_t, q_t in zip(gates.unbind(1), k.unbind(1), v.unbind(1), q.unbind(1)):
        g = g_t[:, :, None, None]
        kv = k_t[:, :, :, None] * v_t[:, :, None, :]
        h = g * h + kv
        ys.append((q_t[:, :, :, None] * h).sum(-2))
    return torch.stack(ys, dim=1)
