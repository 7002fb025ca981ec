"""ssd.py — Mamba-2-style head-wise SSD selective scan (checkpoint + recompute).

Host side of the SSD plug-in (reference mlx_recurrence/ssd.py).  Per head
``head`` and channel ``d`` the state is ``h[b, head, d, n]``::

    decay    = exp(delta[b,t,head] * A_neg[head,n])
    h[d, n]  = decay * h[d, n] + delta[b,t,head] * B[b,t,head,n] * u[b,t,head,d]
    y[b,t,head,d] = sum_n h[d, n] * C[b,t,head,n]

Public API (reference ssd.py:344-394):
    ssd_scan(u, delta, B, C, A_neg, seg=32)              -> y [B, L, H, Dh] fp32
    ssd_scan_with_state(u, delta, B, C, A_neg, seg=32)   -> (y, final_state [B, H, Dh, N])
    ssd_scan_reference(u, delta, B, C, A_neg)            -> y (per-step torch loop)

``A_neg`` is [H, N] as in the reference (ssd.py:62); a per-head A (Mamba-2)
is passed either as ``A[:, None].expand(H, N)`` (its gradient then sums over n
through autograd) or, beyond the reference, as the [H] vector itself (the
gradient is then [H]).  Beyond the reference: keyword-only ``initial_state``
[B, H, Dh, N] and the gradient of a loss that uses ``final_state`` (the
reference VJP reads only the cotangent of y, ssd.py:334).
"""
from __future__ import annotations

import torch

from . import _lib
from ._chassis import DEFAULT_SEG, check_segment_shape


def _validate(u, delta, B, C, A_neg):
    if u.ndim != 4:
        raise ValueError(f"u must be [B, L, H, Dh], got shape {tuple(u.shape)}")
    Bsz, L, H, Dh = u.shape
    if A_neg.ndim not in (1, 2) or A_neg.shape[0] != H:
        raise ValueError(f"A_neg must be [H, N] (or [H], one rate per head) with H={H}, got {tuple(A_neg.shape)}")
    N = A_neg.shape[1] if A_neg.ndim == 2 else B.shape[-1]
    if tuple(delta.shape) != (Bsz, L, H):
        raise ValueError(f"delta must be [B, L, H] = [{Bsz}, {L}, {H}], got {tuple(delta.shape)}")
    for name, t in (("B", B), ("C", C)):
        if tuple(t.shape) != (Bsz, L, H, N):
            raise ValueError(f"{name} must be [B, L, H, N] = [{Bsz}, {L}, {H}, {N}], got {tuple(t.shape)}")
    return Bsz, L, H, Dh, N


def _decay_rates(A_neg):
    """fp32 decay rates for the kernels and their layout flag.

    An ``A_neg`` that is one rate per head broadcast over N (stride 0 along N,
    e.g. ``A[:, None].expand(H, N)``) is passed as the [H] vector with flag 0,
    which selects the chunked MFMA kernels; any other [H, N] array is passed
    dense with flag 1.  Both give the same results; the gradient is [H, N].
    A 1-D A_neg [H] is the per-head vector itself."""
    if A_neg.ndim == 1:
        return _lib.prep(A_neg, torch.float32), 0
    if A_neg.shape[1] > 1 and A_neg.stride(1) == 0:
        return _lib.prep(A_neg[:, 0], torch.float32), 0
    return _lib.prep(A_neg, torch.float32), 1


class _SSDScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, delta, Bm, Cm, A_neg, h0, seg):
        dev = _lib.require_device(u, delta, Bm, Cm, A_neg, h0)
        dt = _lib.common_dtype(u, delta, Bm, Cm)
        u_, d_, B_, C_ = (_lib.prep(t, dt) for t in (u, delta, Bm, Cm))
        A_, a_sn = _decay_rates(A_neg)
        Bsz, L, H, Dh = u_.shape
        N = B_.shape[-1]
        h0_ = None if h0 is None else _lib.prep(h0, torch.float32)
        nC = L // _lib.chunk_len(L, seg)
        y = torch.empty((Bsz, L, H, Dh), dtype=torch.float32, device=dev)
        ckpt = torch.empty((Bsz, H, nC, Dh, N), dtype=torch.float32, device=dev)
        with _lib.device_guard(dev):
            ws = _lib.ssd_workspace(Bsz, L, H, Dh, N, seg, a_sn, dt, 0, dev)
            _lib.ssd_fwd(u_, d_, B_, C_, A_, a_sn, h0_, seg, y, ckpt, ws)
        ctx.save_for_backward(u_, d_, B_, C_, A_, h0_, ckpt)
        ctx.seg = seg
        ctx.a_sn = a_sn
        ctx.a_dim = A_neg.ndim
        ctx.set_materialize_grads(False)
        return y, ckpt[:, :, -1]

    @staticmethod
    def backward(ctx, dy, dfinal):
        u_, d_, B_, C_, A_, h0_, ckpt = ctx.saved_tensors
        Bsz, L, H, Dh = u_.shape
        N = B_.shape[-1]
        dev = u_.device
        dy = torch.zeros((Bsz, L, H, Dh), dtype=torch.float32, device=dev) if dy is None else _lib.prep(dy, torch.float32)
        dfinal = None if dfinal is None else _lib.prep(dfinal, torch.float32)
        du, dd, dB, dC = (torch.empty_like(t) for t in (u_, d_, B_, C_))
        # [H]: the library sums the gradient over n itself (one rate per head)
        dA = torch.empty((H,) if ctx.a_dim == 1 else (H, N), dtype=torch.float32, device=dev)
        dh0 = torch.empty((Bsz, H, Dh, N), dtype=torch.float32, device=dev) if ctx.needs_input_grad[5] else None
        with _lib.device_guard(dev):
            ws = _lib.ssd_workspace(Bsz, L, H, Dh, N, ctx.seg, ctx.a_sn, u_.dtype, 1, dev)
            _lib.ssd_bwd(dy, dfinal, u_, d_, B_, C_, A_, ctx.a_sn, h0_, ckpt, ctx.seg, du, dd, dB, dC, dA, dh0, ws)
        return du, dd, dB, dC, dA, dh0, None


def _run(u, delta, B, C, A_neg, seg, initial_state):
    Bsz, L, H, Dh, N = _validate(u, delta, B, C, A_neg)
    check_segment_shape(L, seg, Dh, "Dh")
    if initial_state is not None and tuple(initial_state.shape) != (Bsz, H, Dh, N):
        raise ValueError(
            f"initial_state must be [B, H, Dh, N] = [{Bsz}, {H}, {Dh}, {N}], got {tuple(initial_state.shape)}"
        )
    ext = _lib.autograd_ext()
    if ext is not None:   # the same forward / backward as one C++ autograd node
        return ext.ssd_scan(u, delta, B, C, A_neg, initial_state, seg)
    return _SSDScan.apply(u, delta, B, C, A_neg, initial_state, seg)


def ssd_scan(u, delta, B, C, A_neg, seg=DEFAULT_SEG, *, initial_state=None):
    """Head-wise SSD (Mamba-2) selective scan on the GPU (fused forward + backward).

    Args:
        u:      [B, L, H, Dh]   input projected to heads x channels
        delta:  [B, L, H]       per-token, per-head step size
        B:      [B, L, H, N]    input projection
        C:      [B, L, H, N]    output projection
        A_neg:  [H, N]          decay rates (negative); [H] for one rate per head
        seg:    checkpoint segment length (L % seg == 0; default 32)

    Returns:
        y:      [B, L, H, Dh] float32

    ``Dh`` must be a multiple of 32.  fp32 state/accumulation internally.
    """
    y, _ = _run(u, delta, B, C, A_neg, seg, initial_state)
    return y


def ssd_scan_with_state(u, delta, B, C, A_neg, seg=DEFAULT_SEG, *, initial_state=None):
    """SSD scan that also returns the final per-head state [B, H, Dh, N]."""
    return _run(u, delta, B, C, A_neg, seg, initial_state)


def ssd_scan_reference(u, delta, B, C, A_neg, *, initial_state=None):
    """Per-step torch loop, op for op as the reference's ssd_scan_reference
    (ssd.py:382-394).  Differentiable; runs on any device."""
    Bsz, L, H, Dh = u.shape
    N = B.shape[-1]
    if A_neg.ndim == 1:   # one rate per head
        A_neg = A_neg[:, None].expand(H, N)
    ct = torch.float32
    for t in (u, delta, B, C, A_neg):
        ct = torch.promote_types(ct, t.dtype)
    u, delta, B, C, A_neg = (t.to(ct) for t in (u, delta, B, C, A_neg))
    h = torch.zeros((Bsz, H, Dh, N), dtype=ct, device=u.device) if initial_state is None else initial_state.to(ct)
    ys = []
    # the per-step slices come from unbind (one backward stack for all steps,
    # where indexing [:, t] would scatter a full-size gradient per step)
    for dl_t, B_t, C_t, u_t in zip(delta.unbind(1), B.unbind(1), C.unbind(1), u.unbind(1)):
        dt = dl_t[:, :, None, None]
        decay = torch.exp(dt * A_neg[None, :, None, :])
        inp = dt * B_t[:, :, None, :] * u_t[:, :, :, None]
        h = decay * h + inp
        ys.append((h * C_t[:, :, None, :]).sum(-1))
    return torch.stack(ys, dim=1)
