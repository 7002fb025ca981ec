"""gdn.py — Gated DeltaNet recurrence (checkpoint + recompute), the reference's
designed next plug-in (docs/DESIGN_gated_deltanet.md; not code in the
reference).  Per (batch, head) the state is S [Dh(i), Dh(j)]::

    S_t = alpha_t (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T
        = alpha_t S_{t-1} - alpha_t beta_t k_t (k_t^T S_{t-1}) + beta_t k_t v_t^T
    o_t = S_t^T q_t            (o_t[j] = sum_i q_t[i] S_t[i, j], the post-update state)

with the reference's pinned convention (DESIGN_gated_deltanet.md:56-90, (R1'')
and (R2'): k and q on the row axis i, v and o on the column axis j) and its
input contract (:461-464, :552-555): q and k are L2-normalised by the caller,
alpha and beta come pre-activated ([B, L, H], alpha = exp(a) in (0, 1],
beta = sigmoid(b)).

Public API (mirroring gla.py's):
    gated_deltanet_scan(q, k, v, alpha, beta, seg=32)             -> y [B, L, H, Dh] fp32
    gated_deltanet_scan_with_state(q, k, v, alpha, beta, seg=32)  -> (y, final_state [B, H, Dh, Dh])
    gated_deltanet_reference(q, k, v, alpha, beta)                -> y (per-step torch loop)

Keyword-only ``initial_state`` [B, H, Dh, Dh]; the gradient of a loss on
``final_state`` is honoured.  Shape rules as the other scans: L % seg == 0,
Dh % 32 == 0 (the kernels cover Dh = 32 and 64).
"""
from __future__ import annotations

import torch

from . import _lib
from ._chassis import DEFAULT_SEG, check_segment_shape


def _validate(q, k, v, alpha, beta):
    if q.ndim != 4:
        raise ValueError(f"q must be [B, L, H, Dh], got shape {tuple(q.shape)}")
    B, L, H, Dh = q.shape
    for name, t in (("k", k), ("v", v)):
        if tuple(t.shape) != (B, L, H, Dh):
            raise ValueError(f"{name} must be [B, L, H, Dh] = [{B}, {L}, {H}, {Dh}], got {tuple(t.shape)}")
    for name, t in (("alpha", alpha), ("beta", beta)):
        if tuple(t.shape) != (B, L, H):
            raise ValueError(f"{name} must be [B, L, H] = [{B}, {L}, {H}], got {tuple(t.shape)}")
    return B, L, H, Dh


class _GDNScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, alpha, beta, h0, seg):
        dev = _lib.require_device(q, k, v, alpha, beta, h0)
        dt = _lib.common_dtype(q, k, v, alpha, beta)
        q_, k_, v_, a_, b_ = (_lib.prep(t, dt) for t in (q, k, v, alpha, beta))
        B, L, H, Dh = q_.shape
        h0_ = None if h0 is None else _lib.prep(h0, torch.float32)
        nC = L // _lib.chunk_len(L, seg)
        y = torch.empty((B, L, H, Dh), dtype=torch.float32, device=dev)
        ckpt = torch.empty((B, H, nC, Dh, Dh), dtype=torch.float32, device=dev)
        with _lib.device_guard(dev):
            ws = _lib.gdn_fwd_workspace(B, L, H, Dh, seg, q_.dtype, dev)
            _lib.gdn_fwd(q_, k_, v_, a_, b_, h0_, seg, y, ckpt, ws)
        ctx.save_for_backward(q_, k_, v_, a_, b_, h0_, ckpt)
        ctx.seg = seg
        ctx.set_materialize_grads(False)
        return y, ckpt[:, :, -1]

    @staticmethod
    def backward(ctx, dy, dfinal):
        q_, k_, v_, a_, b_, h0_, ckpt = ctx.saved_tensors
        B, L, H, Dh = q_.shape
        dev = q_.device
        dy = torch.zeros((B, L, H, Dh), dtype=torch.float32, device=dev) if dy is None else _lib.prep(dy, torch.float32)
        dfinal = None if dfinal is None else _lib.prep(dfinal, torch.float32)
        dq, dk, dv, da, db = (torch.empty_like(t) for t in (q_, k_, v_, a_, b_))
        dh0 = torch.empty((B, H, Dh, Dh), dtype=torch.float32, device=dev) if ctx.needs_input_grad[5] else None
        with _lib.device_guard(dev):
            ws = _lib.gdn_workspace(B, L, H, Dh, ctx.seg, q_.dtype, dev)
            _lib.gdn_bwd(dy, dfinal, q_, k_, v_, a_, b_, h0_, ckpt, ctx.seg, dq, dk, dv, da, db, dh0, ws)
        return dq, dk, dv, da, db, dh0, None


def _run(q, k, v, alpha, beta, seg, initial_state):
    B, L, H, Dh = _validate(q, k, v, alpha, beta)
    check_segment_shape(L, seg, Dh, "Dh")
    if initial_state is not None and tuple(initial_state.shape) != (B, H, Dh, Dh):
        raise ValueError(
            f"initial_state must be [B, H, Dh, Dh] = [{B}, {H}, {Dh}, {Dh}], got {tuple(initial_state.shape)}"
        )
    return _GDNScan.apply(q, k, v, alpha, beta, initial_state, seg)


def gated_deltanet_scan(q, k, v, alpha, beta, seg=DEFAULT_SEG, *, initial_state=None):
    """Gated DeltaNet scan on the GPU (fused forward + backward).

    Args:
        q, k:   [B, L, H, Dh]  query / key, L2-normalised over Dh by the caller
        v:      [B, L, H, Dh]  value
        alpha:  [B, L, H]      decay gate in (0, 1] (exp of a non-positive logit)
        beta:   [B, L, H]      write strength in (0, 1) (sigmoid of a logit)
        seg:    checkpoint segment length (L % seg == 0; default 32)

    Returns:
        y:      [B, L, H, Dh] float32

    ``Dh`` must be a multiple of 32 (32 and 64 run on the kernels).  fp32
    state/accumulation internally.
    """
    y, _ = _run(q, k, v, alpha, beta, seg, initial_state)
    return y


def gated_deltanet_scan_with_state(q, k, v, alpha, beta, seg=DEFAULT_SEG, *, initial_state=None):
    """Gated DeltaNet scan that also returns the final state S [B, H, Dh(i), Dh(j)]."""
    return _run(q, k, v, alpha, beta, seg, initial_state)


def gated_deltanet_reference(q, k, v, alpha, beta, *, initial_state=None):
    """Per-step torch loop of the recurrence (R1'') and output (R2') of
    DESIGN_gated_deltanet.md:56-90, the counterpart of the reference's planned
    gated_deltanet_reference (:520-521).  Differentiable; runs on any device."""
    B, L, H, Dh = q.shape
    ct = torch.float32
    for t in (q, k, v, alpha, beta):
        ct = torch.promote_types(ct, t.dtype)
    q, k, v, alpha, beta = (t.to(ct) for t in (q, k, v, alpha, beta))
    S = torch.zeros((B, H, Dh, Dh), dtype=ct, device=q.device) if initial_state is None else initial_state.to(ct)
    ys = []
    for q_t, k_t, v_t, a_t, b_t in zip(q.unbind(1), k.unbind(1), v.unbind(1), alpha.unbind(1), beta.unbind(1)):
        a, b = a_t[:, :, None, None], b_t[:, :, None, None]
        p = (k_t[:, :, :, None] * S).sum(-2)                                 # k^T S_{t-1}  [B,H,Dh(j)]
        S = a * (S - b * k_t[:, :, :, None] * p[:, :, None, :]) + b * k_t[:, :, :, None] * v_t[:, :, None, :]
        ys.append((q_t[:, :, :, None] * S).sum(-2))                          # S^T q
    return torch.stack(ys, dim=1)
