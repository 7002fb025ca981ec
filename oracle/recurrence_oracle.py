"""Float64 CPU oracle for the four scans — TEST INFRASTRUCTURE ONLY.

This module is the checker the GPU kernels are compared against.  Only the
tests (tests/), ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import it; the product path (mlx_recurrence_amd) never does.

It restates, in float64 NumPy, the reference's per-step recurrences and their
adjoints (D-CSIL/mlx-recurrence v0.3.0):

  SSD     forward ssd.py:382-394 (kernel ssd.py:85-111), final state
          ssd.py:365-375, adjoint ssd.py:203-268
  GLA     forward gla.py:336-346 (kernel gla.py:78-100), final state
          gla.py:321-329, adjoint gla.py:184-236
  RG-LRU  forward rglru.py:274-282, adjoint rglru.py:36-39 and :166-180
  rotLRU  forward rotlru.py:338-351, adjoint rotlru.py:317-322 and :205-235
  Gated DeltaNet (the reference's designed next plug-in, not code there):
          recurrence and output docs/DESIGN_gated_deltanet.md:56-90 (R1'',
          R2'), adjoint :334-440 (B0, Bq, Bp', Bv, grad_k terms A + B, Bbeta,
          Balpha)

Extensions beyond the reference, present in the kernels and checked here:
an optional initial state h0 and a cotangent ``dfinal`` on the final state
(the reference VJPs read only the cotangent of y).  With h0=None and
dfinal=None the functions are exactly the reference semantics.

How each function is pinned (tests/test_oracle.py) — the reference ships no
golden vectors, so the oracle is checked against mathematics it must agree
with, chosen so that a dropped term, a wrong sign or a transposed operand
fails at least one check:
  * forward: closed forms (RG-LRU with constant a = discounted sum; GLA with
    g = 1 = causal linear attention as one masked matmul; SSD = the Mamba-2
    quadratic "dual" form, per state n), the reference's chunked cumsum form
    (legacy/_utils.py:27-61), the invariants of the reference tests
    (theta = 0 rotLRU = RG-LRU, pure rotation preserves the pair norm,
    final state = y[:, -1]), and brute force on tiny inputs;
  * backward: float64 central finite differences of the forward on every
    input (method of tests/test_backward_metal.py:179-238), and torch float64
    autograd of an independently written per-step loop.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "ssd_forward",
    "ssd_backward",
    "gla_forward",
    "gla_backward",
    "rglru_forward",
    "rglru_backward",
    "rglru_gates",
    "rglru_gated_forward",
    "rglru_gated_backward",
    "rotlru_forward",
    "rotlru_backward",
    "rotlru_theta_forward",
    "rotlru_theta_backward",
    "ssd_dual_form",
    "gla_causal_linear_attention",
    "rglru_discounted_sum",
    "chunked_cumsum_scan",
    "gdn_forward",
    "gdn_backward",
]


def _f64(*arrs):
    return [None if a is None else np.asarray(a, dtype=np.float64) for a in arrs]


# ---------------------------------------------------------------------- SSD
def _ssd_states(u, delta, Bm, Cm, A_neg, h0):
    Bsz, L, H, Dh = u.shape
    N = A_neg.shape[-1]
    hs = np.empty((L + 1, Bsz, H, Dh, N))
    hs[0] = 0.0 if h0 is None else h0
    y = np.empty((Bsz, L, H, Dh))
    for t in range(L):
        dt = delta[:, t, :, None, None]                             # [B,H,1,1]
        decay = np.exp(dt * A_neg[None, :, None, :])                # [B,H,1,N]
        inp = dt * Bm[:, t, :, None, :] * u[:, t, :, :, None]       # [B,H,Dh,N]
        hs[t + 1] = decay * hs[t] + inp
        y[:, t] = (hs[t + 1] * Cm[:, t, :, None, :]).sum(-1)
    return y, hs


def ssd_forward(u, delta, Bm, Cm, A_neg, h0=None):
    """y [B,L,H,Dh] and final state [B,H,Dh,N] (ssd.py:382-394, :372-375)."""
    u, delta, Bm, Cm, A_neg, h0 = _f64(u, delta, Bm, Cm, A_neg, h0)
    y, hs = _ssd_states(u, delta, Bm, Cm, A_neg, h0)
    return y, hs[-1].copy()


def ssd_backward(dy, u, delta, Bm, Cm, A_neg, h0=None, dfinal=None):
    """Explicit float64 adjoint sweep (ssd.py:203-268, then the host sums
    ssd.py:302-305).  Returns (du, ddelta, dB, dC, dA_neg, dh0)."""
    dy, u, delta, Bm, Cm, A_neg, h0, dfinal = _f64(dy, u, delta, Bm, Cm, A_neg, h0, dfinal)
    Bsz, L, H, Dh = u.shape
    N = A_neg.shape[-1]
    _, hs = _ssd_states(u, delta, Bm, Cm, A_neg, h0)
    lam = np.zeros((Bsz, H, Dh, N)) if dfinal is None else dfinal.copy()
    du = np.empty_like(u)
    dd = np.empty_like(delta)
    dB = np.empty_like(Bm)
    dC = np.empty_like(Cm)
    dA = np.zeros_like(A_neg)
    A = A_neg[None, :, None, :]
    for t in range(L - 1, -1, -1):
        dt = delta[:, t, :, None, None]
        decay = np.exp(dt * A)
        hprev, hcur = hs[t], hs[t + 1]
        bt = Bm[:, t, :, None, :]
        ut = u[:, t, :, :, None]
        lam = lam + dy[:, t, :, :, None] * Cm[:, t, :, None, :]     # ssd.py:237
        du[:, t] = (lam * dt * bt).sum(-1)                          # :239
        dd[:, t] = (lam * (A * decay * hprev + bt * ut)).sum((-1, -2))  # :240
        dA += (lam * dt * decay * hprev).sum((0, 2))                # :241, :305
        dB[:, t] = (lam * dt * ut).sum(-2)                          # :244
        dC[:, t] = (hcur * dy[:, t, :, :, None]).sum(-2)            # :245
        lam = lam * decay                                           # :252
    return du, dd, dB, dC, dA, lam


def ssd_dual_form(u, delta, Bm, Cm, A_neg, h0=None):
    """Closed form of the SSD forward (Mamba-2 quadratic 'dual' form, per n):
    y_t[d] = sum_n C_t[n] ( sum_{s<=t} exp(A[n] (cum_t - cum_s)) delta_s B_s[n] u_s[d]
                            + exp(A[n] cum_t) h0[d, n] ),  cum_t = sum_{r<=t} delta_r.
    An independent check of ssd_forward (no recurrence)."""
    u, delta, Bm, Cm, A_neg, h0 = _f64(u, delta, Bm, Cm, A_neg, h0)
    Bsz, L, H, Dh = u.shape
    cum = np.cumsum(delta, axis=1)                                  # [B,L,H]
    diff = cum[:, :, None, :] - cum[:, None, :, :]                  # [B,t,s,H]
    mask = np.tril(np.ones((L, L), dtype=bool))[None, :, :, None]
    # decay[b,t,s,h,n] = exp(A[h,n] * (cum_t - cum_s)) for s <= t
    dec = np.where(mask[..., None], np.exp(diff[..., None] * A_neg[None, None, None]), 0.0)
    w = dec * (delta[:, None, :, :, None] * Bm[:, None, :, :, :])   # [B,t,s,H,N]
    w = w * Cm[:, :, None, :, :]
    M = w.sum(-1)                                                   # [B,t,s,H]
    y = np.einsum("btsh,bshd->bthd", M, u)
    if h0 is not None:
        q = np.exp(cum[..., None] * A_neg[None, None])              # [B,L,H,N]
        y = y + np.einsum("bthn,bhdn->bthd", Cm * q, h0)
    return y


# ---------------------------------------------------------------------- GLA
def _gla_states(q, k, v, g, h0):
    B, L, H, Dh = q.shape
    hs = np.empty((L + 1, B, H, Dh, Dh))
    hs[0] = 0.0 if h0 is None else h0
    y = np.empty((B, L, H, Dh))
    for t in range(L):
        gt = g[:, t, :, None, None]
        kv = k[:, t, :, :, None] * v[:, t, :, None, :]
        hs[t + 1] = gt * hs[t] + kv
        y[:, t] = (q[:, t, :, :, None] * hs[t + 1]).sum(-2)
    return y, hs


def gla_forward(q, k, v, gates, h0=None):
    """y [B,L,H,Dh] and final state S [B,H,Dh(i),Dh(j)] (gla.py:336-346, :328-329)."""
    q, k, v, gates, h0 = _f64(q, k, v, gates, h0)
    y, hs = _gla_states(q, k, v, gates, h0)
    return y, hs[-1].copy()


def gla_backward(dy, q, k, v, gates, h0=None, dfinal=None):
    """Explicit float64 adjoint sweep (gla.py:184-236 and the sums :266-268).
    Returns (dq, dk, dv, dgates, dh0)."""
    dy, q, k, v, gates, h0, dfinal = _f64(dy, q, k, v, gates, h0, dfinal)
    B, L, H, Dh = q.shape
    _, hs = _gla_states(q, k, v, gates, h0)
    lam = np.zeros((B, H, Dh, Dh)) if dfinal is None else dfinal.copy()
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    dg = np.empty_like(gates)
    for t in range(L - 1, -1, -1):
        go = dy[:, t, :, None, :]                                   # [B,H,1,Dh(j)]
        lam = lam + q[:, t, :, :, None] * go                        # gla.py:213
        dq[:, t] = (go * hs[t + 1]).sum(-1)                         # :219
        dk[:, t] = (lam * v[:, t, :, None, :]).sum(-1)              # :220
        dv[:, t] = (lam * k[:, t, :, :, None]).sum(-2)              # :215
        dg[:, t] = (lam * hs[t]).sum((-1, -2))                      # :216
        lam = lam * gates[:, t, :, None, None]                      # :227
    return dq, dk, dv, dg, lam


def gla_causal_linear_attention(q, k, v):
    """Closed form of the GLA forward with g = 1 and zero initial state:
    o_t = sum_{s<=t} (q_t . k_s) v_s, one masked matmul per (b, h)."""
    q, k, v = _f64(q, k, v)
    L = q.shape[1]
    scores = np.einsum("bthi,bshi->bhts", q, k)
    scores = scores * np.tril(np.ones((L, L)))[None, None]
    return np.einsum("bhts,bshj->bthj", scores, v)


# ------------------------------------------------------------------- RG-LRU
def rglru_forward(a, x, h0=None):
    """y [B,L,D] and final state [B,D] (rglru.py:274-282, :266-267)."""
    a, x, h0 = _f64(a, x, h0)
    B, L, D = a.shape
    h = np.zeros((B, D)) if h0 is None else h0.copy()
    y = np.empty((B, L, D))
    for t in range(L):
        h = a[:, t] * h + x[:, t]
        y[:, t] = h
    return y, h.copy()


def rglru_backward(dy, a, x, h0=None, dfinal=None):
    """Explicit adjoint (rglru.py:36-39, :173-178). Returns (da, dx, dh0)."""
    dy, a, x, h0, dfinal = _f64(dy, a, x, h0, dfinal)
    B, L, D = a.shape
    y, _ = rglru_forward(a, x, h0)
    hprev = np.concatenate([(np.zeros((B, 1, D)) if h0 is None else h0[:, None]), y[:, :-1]], axis=1)
    lam = np.zeros((B, D)) if dfinal is None else dfinal.copy()
    da, dx = np.empty_like(a), np.empty_like(x)
    for t in range(L - 1, -1, -1):
        lam = lam + dy[:, t]
        dx[:, t] = lam
        da[:, t] = lam * hprev[:, t]
        lam = lam * a[:, t]
    return da, dx, lam


def rglru_gates(r, i, x, lam, c=8.0):
    """RG-LRU gate math (rglru.py:13-14, the Griffin formulas the reference
    leaves to MLX host code, rglru.py:19-27): a = exp(-c softplus(lam)
    sigmoid(r)), x' = sqrt(1 - a^2) (i x).  lam is per channel [D]."""
    r, i, x, lam = _f64(r, i, x, lam)
    sp = np.logaddexp(0.0, lam)
    sr = 1.0 / (1.0 + np.exp(-r))
    a = np.exp(-c * sp * sr)
    return a, np.sqrt(1.0 - a * a) * (i * x)


def rglru_gated_forward(r, i, x, lam, c=8.0, h0=None):
    """Scan of the gated inputs: rglru_forward(*rglru_gates(...), h0)."""
    a, xg = rglru_gates(r, i, x, lam, c)
    return rglru_forward(a, xg, h0)


def rglru_gated_backward(dy, r, i, x, lam, c=8.0, h0=None, dfinal=None):
    """Chain rule of rglru_gates through rglru_backward.
    Returns (dr, di, dx, dlam [D], dh0)."""
    r, i, x, lam = _f64(r, i, x, lam)
    a, xg = rglru_gates(r, i, x, lam, c)
    da, dxg, dh0 = rglru_backward(dy, a, xg, h0, dfinal)
    sp = np.logaddexp(0.0, lam)
    sr = 1.0 / (1.0 + np.exp(-r))
    s = np.sqrt(1.0 - a * a)
    # x' = s (i x): d/ds, d/di, d/dx; s = sqrt(1 - a^2): ds/da = -a / s
    ds = dxg * i * x
    dz = (da - ds * a / s) * a                 # a = exp(z), z = -c sp sr
    dr = dz * (-c * sp) * sr * (1.0 - sr)
    dlam = (dz * (-c * sr)).sum(axis=(0, 1)) / (1.0 + np.exp(-lam))
    return dr, dxg * s * x, dxg * s * i, dlam, dh0


def rglru_discounted_sum(a_const, x):
    """Closed form for a constant gate: y_t = sum_{s<=t} a^(t-s) x_s."""
    (x,) = _f64(x)
    L = x.shape[1]
    p = np.arange(L)
    W = np.where(p[:, None] >= p[None, :], float(a_const) ** (p[:, None] - p[None, :]).clip(min=0), 0.0)
    return np.einsum("ts,bsd->btd", W, x)


def chunked_cumsum_scan(decay, inp, chunk=32):
    """The reference's chunked closed form h_t = P_t (h_prev + cumsum(inp / P))
    with P the in-chunk cumulative product of decay (legacy/_utils.py:27-61),
    in float64 without its epsilon guards.  decay must be nonzero."""
    decay, inp = _f64(decay, inp)
    B, L, D = decay.shape
    out = np.empty_like(inp)
    h_prev = np.zeros((B, 1, D))
    for t0 in range(0, L, chunk):
        t1 = min(t0 + chunk, L)
        P = np.cumprod(decay[:, t0:t1], axis=1)
        hc = P * (h_prev + np.cumsum(inp[:, t0:t1] / P, axis=1))
        out[:, t0:t1] = hc
        h_prev = hc[:, -1:]
    return out


# ------------------------------------------------------------------- rotLRU
def rotlru_forward(a, cs, sn, x, h0=None):
    """y [B,L,2Dp] (interleaved) and final state [B,2Dp] (rotlru.py:338-351)."""
    a, cs, sn, x, h0 = _f64(a, cs, sn, x, h0)
    B, L, Dp = a.shape
    xp = x.reshape(B, L, Dp, 2)
    if h0 is None:
        u = np.zeros((B, Dp))
        w = np.zeros((B, Dp))
    else:
        u, w = h0.reshape(B, Dp, 2)[..., 0].copy(), h0.reshape(B, Dp, 2)[..., 1].copy()
    y = np.empty((B, L, Dp, 2))
    for t in range(L):
        at, c, s = a[:, t], cs[:, t], sn[:, t]
        un = at * (c * u - s * w) + xp[:, t, :, 0]
        wn = at * (s * u + c * w) + xp[:, t, :, 1]
        u, w = un, wn
        y[:, t, :, 0] = u
        y[:, t, :, 1] = w
    y = y.reshape(B, L, 2 * Dp)
    return y, y[:, -1].copy()


def rotlru_theta_forward(a, theta, x, h0=None):
    """rotLRU with the rotation as its angle (cos / sin of rotlru.py:18-23)."""
    theta = np.asarray(theta, dtype=np.float64)
    return rotlru_forward(a, np.cos(theta), np.sin(theta), x, h0)


def rotlru_theta_backward(dy, a, theta, x, h0=None, dfinal=None):
    """Chain rule of (cos, sin) through rotlru_backward: (da, dtheta, dx, dh0)."""
    theta = np.asarray(theta, dtype=np.float64)
    da, dcs, dsn, dx, dh0 = rotlru_backward(dy, a, np.cos(theta), np.sin(theta), x, h0, dfinal)
    return da, np.cos(theta) * dsn - np.sin(theta) * dcs, dx, dh0


def rotlru_backward(dy, a, cs, sn, x, h0=None, dfinal=None):
    """Explicit adjoint (rotlru.py:317-322, :212-234).
    Returns (da, dcs, dsn, dx, dh0)."""
    dy, a, cs, sn, x, h0, dfinal = _f64(dy, a, cs, sn, x, h0, dfinal)
    B, L, Dp = a.shape
    y, _ = rotlru_forward(a, cs, sn, x, h0)
    yp = y.reshape(B, L, Dp, 2)
    h0p = np.zeros((B, Dp, 2)) if h0 is None else h0.reshape(B, Dp, 2)
    gp = dy.reshape(B, L, Dp, 2)
    if dfinal is None:
        lu, lw = np.zeros((B, Dp)), np.zeros((B, Dp))
    else:
        lu, lw = dfinal.reshape(B, Dp, 2)[..., 0].copy(), dfinal.reshape(B, Dp, 2)[..., 1].copy()
    da, dcs, dsn = np.empty_like(a), np.empty_like(cs), np.empty_like(sn)
    dx = np.empty((B, L, Dp, 2))
    for t in range(L - 1, -1, -1):
        up, wp = (yp[:, t - 1, :, 0], yp[:, t - 1, :, 1]) if t > 0 else (h0p[..., 0], h0p[..., 1])
        at, c, s = a[:, t], cs[:, t], sn[:, t]
        lu = lu + gp[:, t, :, 0]
        lw = lw + gp[:, t, :, 1]
        dx[:, t, :, 0] = lu
        dx[:, t, :, 1] = lw
        ru = c * up - s * wp
        rw = s * up + c * wp
        da[:, t] = lu * ru + lw * rw
        dcs[:, t] = at * (lu * up + lw * wp)
        dsn[:, t] = at * (lw * up - lu * wp)
        lu, lw = at * (c * lu + s * lw), at * (-s * lu + c * lw)
    dh0 = np.stack([lu, lw], axis=-1).reshape(B, 2 * Dp)
    return da, dcs, dsn, dx.reshape(B, L, 2 * Dp), dh0


# ------------------------------------------------------------ Gated DeltaNet
def _gdn_states(q, k, v, alpha, beta, h0):
    B, L, H, Dh = q.shape
    hs = np.empty((L + 1, B, H, Dh, Dh))
    hs[0] = 0.0 if h0 is None else h0
    y = np.empty((B, L, H, Dh))
    for t in range(L):
        kt, vt = k[:, t], v[:, t]                                   # [B,H,Dh]
        a, b = alpha[:, t, :, None, None], beta[:, t, :, None, None]
        p = np.einsum("bhi,bhij->bhj", kt, hs[t])                   # k^T S_{t-1}
        hs[t + 1] = a * (hs[t] - b * kt[..., :, None] * p[..., None, :]) + b * kt[..., :, None] * vt[..., None, :]
        y[:, t] = np.einsum("bhi,bhij->bhj", q[:, t], hs[t + 1])     # o_t = S_t^T q_t
    return y, hs


def gdn_forward(q, k, v, alpha, beta, h0=None):
    """Gated DeltaNet, per (b, h): S_t = alpha_t (I - beta_t k_t k_t^T) S_{t-1}
    + beta_t k_t v_t^T, o_t = S_t^T q_t (DESIGN_gated_deltanet.md:56-90, the
    reference's pinned convention: S[i, j], k and q on the row axis i, v and o
    on the column axis j).  q, k, v [B,L,H,Dh], alpha, beta [B,L,H] (already
    activated).  Returns y [B,L,H,Dh] and the final state [B,H,Dh(i),Dh(j)]."""
    q, k, v, alpha, beta, h0 = _f64(q, k, v, alpha, beta, h0)
    y, hs = _gdn_states(q, k, v, alpha, beta, h0)
    return y, hs[-1].copy()


def gdn_backward(dy, q, k, v, alpha, beta, h0=None, dfinal=None):
    """Explicit float64 adjoint (DESIGN_gated_deltanet.md:334-440), newest to
    oldest with dS the adjoint of S_t:
      dS += q_t go_t^T;  dq_t = S_t go_t;  d = k_t^T dS;  p = k_t^T S_{t-1};
      dv_t = beta d;  dk_t = dS (beta v - alpha beta p) - alpha beta S_{t-1} d;
      dbeta_t = d . (v - alpha p);  dalpha_t = <dS, S_{t-1}> - beta d . p;
      dS <- alpha (dS - beta k_t d^T).
    Returns (dq, dk, dv, dalpha, dbeta, dh0)."""
    dy, q, k, v, alpha, beta, h0, dfinal = _f64(dy, q, k, v, alpha, beta, h0, dfinal)
    B, L, H, Dh = q.shape
    _, hs = _gdn_states(q, k, v, alpha, beta, h0)
    lam = np.zeros((B, H, Dh, Dh)) if dfinal is None else dfinal.copy()
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    da, db = np.empty_like(alpha), np.empty_like(beta)
    for t in range(L - 1, -1, -1):
        kt, vt, go = k[:, t], v[:, t], dy[:, t]
        a, b = alpha[:, t, :, None], beta[:, t, :, None]            # [B,H,1]
        sp, sc = hs[t], hs[t + 1]
        lam = lam + q[:, t, :, :, None] * go[:, :, None, :]          # (B0)
        dq[:, t] = np.einsum("bhij,bhj->bhi", sc, go)                # (Bq)
        d = np.einsum("bhi,bhij->bhj", kt, lam)
        p = np.einsum("bhi,bhij->bhj", kt, sp)
        dv[:, t] = b * d                                             # (Bv)
        dk[:, t] = np.einsum("bhij,bhj->bhi", lam, b * vt - a * b * p) - a * b * np.einsum("bhij,bhj->bhi", sp, d)
        db[:, t] = (d * (vt - a * p)).sum(-1)                        # (Bbeta)
        da[:, t] = (lam * sp).sum((-1, -2)) - beta[:, t] * (d * p).sum(-1)   # (Balpha)
        lam = a[..., None] * (lam - b[..., None] * kt[..., :, None] * d[..., None, :])   # (Bp')
    return dq, dk, dv, da, db, lam
