"""step.py — single-token decode steps on a cached state (one kernel launch each).

The O(1)-per-token recurrent update that the reference names as its next
inference step (docs/validation/BOTTLENECK_ANALYSIS.md:105-119): each call
advances a cached state by one token, in place, and returns that token's
output.  The states are the final-state layouts of the scans
(``*_scan_with_state``), so a chunked prefill continues directly::

    y, state = mr.ssd_scan_with_state(u, delta, B, C, A_neg)     # prompt
    y_t = mr.ssd_step(u_t, delta_t, B_t, C_t, A_neg, state)      # then per token

    ssd_step(u [B,H,Dh], delta [B,H], B [B,H,N], C [B,H,N], A_neg [H,N] or [H], state [B,H,Dh,N]) -> y [B,H,Dh]
    gla_step(q, k, v [B,H,Dh], gates [B,H], state [B,H,Dh,Dh])                           -> y [B,H,Dh]
    rglru_step(a, x [B,D], state [B,D])                                                   -> y [B,D]
    rotlru_step(a, cs, sn [B,Dp], x [B,2Dp], state [B,2Dp])                               -> y [B,2Dp]

The state must be a contiguous fp32 tensor on the GPU (it is updated in place);
token inputs may be fp32, bf16 or fp16; y is fp32.  Inference only: the steps
are not differentiable, and a call with autograd recording on inputs that
require grad raises.
"""
from __future__ import annotations

import torch

from . import _lib
from .ssd import _decay_rates


def _prepare(name, state, inputs, state_shape, params=()):
    """Device and compute dtype of one step.  The dtype comes from the token
    inputs alone; `params` (SSD's fp32 A_neg) are checked for device and
    autograd but do not promote the token inputs."""
    dev = _lib.require_device(state, *inputs, *params)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (state, *inputs, *params)):
        raise ValueError(f"{name} is not differentiable (inference only); call it under torch.no_grad()")
    if tuple(state.shape) != tuple(state_shape):
        raise ValueError(f"{name}: state must be {list(state_shape)}, got {tuple(state.shape)}")
    if state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError(f"{name}: state must be a contiguous float32 tensor (it is updated in place)")
    dt = _lib.common_dtype(*inputs)
    return dev, dt


def ssd_step(u, delta, B, C, A_neg, state):
    """One SSD token: state[b,h,d,n] = exp(delta A_neg[h,n]) state + delta B[n] u[d];
    returns y[b,h,d] = sum_n state[b,h,d,n] C[n] (reference ssd.py:97-101).
    A_neg is [H, N] or one rate per head [H], as for ssd_scan; the token
    inputs run in their own dtype (A_neg, fp32, does not promote them)."""
    if u.ndim != 3:
        raise ValueError(f"u must be [B, H, Dh], got shape {tuple(u.shape)}")
    Bsz, H, Dh = u.shape
    if B.ndim != 3:
        raise ValueError(f"B must be [B, H, N], got shape {tuple(B.shape)}")
    N = B.shape[-1]
    if A_neg.ndim not in (1, 2) or A_neg.shape[0] != H or (A_neg.ndim == 2 and A_neg.shape[1] != N):
        raise ValueError(f"A_neg must be [H, N] or [H] with H={H}, N={N}, got {tuple(A_neg.shape)}")
    if tuple(delta.shape) != (Bsz, H):
        raise ValueError(f"delta must be [B, H] = [{Bsz}, {H}], got {tuple(delta.shape)}")
    for nm, t in (("B", B), ("C", C)):
        if tuple(t.shape) != (Bsz, H, N):
            raise ValueError(f"{nm} must be [B, H, N] = [{Bsz}, {H}, {N}], got {tuple(t.shape)}")
    dev, dt = _prepare("ssd_step", state, (u, delta, B, C), (Bsz, H, Dh, N), params=(A_neg,))
    u_, d_, B_, C_ = (_lib.prep(t, dt) for t in (u, delta, B, C))
    A_, a_sn = _decay_rates(A_neg)
    y = torch.empty((Bsz, H, Dh), dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        _lib.ssd_step(u_, d_, B_, C_, A_, a_sn, state, y)
    return y


def gla_step(q, k, v, gates, state):
    """One GLA token: state[b,h,i,j] = g state + k[i] v[j]; returns
    y[b,h,j] = sum_i q[i] state[b,h,i,j] (reference gla.py:86-90)."""
    if q.ndim != 3:
        raise ValueError(f"q must be [B, H, Dh], got shape {tuple(q.shape)}")
    Bsz, H, Dh = q.shape
    for nm, t in (("k", k), ("v", v)):
        if tuple(t.shape) != (Bsz, H, Dh):
            raise ValueError(f"{nm} must be [B, H, Dh] = [{Bsz}, {H}, {Dh}], got {tuple(t.shape)}")
    if tuple(gates.shape) != (Bsz, H):
        raise ValueError(f"gates must be [B, H] = [{Bsz}, {H}], got {tuple(gates.shape)}")
    dev, dt = _prepare("gla_step", state, (q, k, v, gates), (Bsz, H, Dh, Dh))
    q_, k_, v_, g_ = (_lib.prep(t, dt) for t in (q, k, v, gates))
    y = torch.empty((Bsz, H, Dh), dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        _lib.gla_step(q_, k_, v_, g_, state, y)
    return y


def rglru_step(a, x, state):
    """One RG-LRU token: state = a state + x; returns the new state
    (reference rglru.py:92; x is the gated input, as for rglru_scan)."""
    if a.ndim != 2 or tuple(x.shape) != tuple(a.shape):
        raise ValueError(f"a and x must both be [B, D], got {tuple(a.shape)} and {tuple(x.shape)}")
    Bsz, D = a.shape
    dev, dt = _prepare("rglru_step", state, (a, x), (Bsz, D))
    a_, x_ = _lib.prep(a, dt), _lib.prep(x, dt)
    y = torch.empty((Bsz, D), dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        _lib.rglru_step(a_, x_, state, y)
    return y


def rotlru_step(a, cs, sn, x, state):
    """One rotLRU token on the interleaved (u, w) pairs: (u, w) = a R(theta)
    (u, w) + (x[2p], x[2p+1]); returns the new state (reference
    rotlru.py:110-111)."""
    if a.ndim != 2 or tuple(cs.shape) != tuple(a.shape) or tuple(sn.shape) != tuple(a.shape):
        raise ValueError(f"a, cs, sn must all be [B, Dp], got {tuple(a.shape)}, {tuple(cs.shape)}, {tuple(sn.shape)}")
    Bsz, Dp = a.shape
    if tuple(x.shape) != (Bsz, 2 * Dp):
        raise ValueError(f"x must be [B, 2*Dp] = [{Bsz}, {2 * Dp}], got {tuple(x.shape)}")
    dev, dt = _prepare("rotlru_step", state, (a, cs, sn, x), (Bsz, 2 * Dp))
    a_, c_, s_, x_ = (_lib.prep(t, dt) for t in (a, cs, sn, x))
    y = torch.empty((Bsz, 2 * Dp), dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        _lib.rotlru_step(a_, c_, s_, x_, state, y)
    return y
