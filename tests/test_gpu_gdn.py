"""GPU parity of the Gated DeltaNet scan (MI355X only).

The HIP forward and backward (rr_gdn_fwd / rr_gdn_bwd through
mr.gated_deltanet_scan_with_state) against the float64 oracle
(orc.gdn_forward / gdn_backward, the recurrence and adjoint of
docs/DESIGN_gated_deltanet.md:56-90 and :334-440) on the same rounded inputs,
at the fp32 bar (1e-5) for fp32 inputs and the 16-bit bar otherwise — tighter
than the reference's own Phase-2 gate (y and gradients within 1e-3,
:532-536).  Size-independent properties at the full bench shape: exact recall
(beta = 1, q = k unit: y = v exactly, whatever alpha and the state), and two
runs agree bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import recurrence_oracle as orc
from tests.gpu_util import TOL, check, rounded, to_dev

import mlx_recurrence_amd as mr

pytestmark = pytest.mark.gpu

F32, BF16, F16 = torch.float32, torch.bfloat16, torch.float16


def _announce(name, **kw):
    print(f"[case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def _inputs(rng, B, L, H, Dh, dist):
    q = _unit(rng.standard_normal((B, L, H, Dh)))
    k = _unit(rng.standard_normal((B, L, H, Dh)))
    v = rng.standard_normal((B, L, H, Dh))
    alpha = np.exp(-rng.uniform(0.01, 0.5, (B, L, H)))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, L, H))))
    if dist == "edges":   # no decay, no write, full write, strong decay
        alpha[:, ::5] = 1.0
        beta[:, ::7] = 0.0
        beta[:, 3::11] = 1.0
        alpha[:, 2::13] = 0.01
    elif dist == "tiny":  # strong decays down to none of the state kept: the dalpha of small alpha
        alpha[:, 3::9] = 1e-4
        alpha[:, 5::11] = 1e-8
        alpha[:, 7::13] = 0.0
    return q, k, v, alpha, beta


def _w(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


GDN_CASES = [
    # (B, L, H, Dh, seg, dtype, dist, h0, dfinal, seed)
    (2, 64, 3, 64, 32, F32, "plain", False, False, 0),
    (1, 96, 2, 32, 16, F32, "plain", True, True, 1),      # T = 16
    (2, 40, 2, 64, 8, F32, "edges", True, True, 2),       # T = 8
    (1, 128, 2, 64, 64, F32, "edges", True, True, 3),     # seg 64: T = 32
    (1, 96, 3, 32, 48, F32, "plain", False, True, 4),     # seg 48: T = 16
    (1, 8, 2, 64, 8, F32, "plain", True, True, 5),        # one interval
    (3, 512, 12, 64, 32, BF16, "plain", False, False, 6),  # bench shape (config 2's B, L, H, Dh)
    (2, 256, 4, 32, 32, F16, "edges", True, True, 7),
    (1, 128, 2, 64, 32, BF16, "edges", True, True, 8),
    # alpha of 1e-4, 1e-8 and 0: dalpha at a strong decay (chunkwise form, then sequential)
    (2, 128, 3, 64, 32, BF16, "tiny", True, True, 9),
    (1, 96, 2, 64, 32, F32, "tiny", True, True, 10),
]


@pytest.mark.parametrize("B,L,H,Dh,seg,dtype,dist,h0,dfinal,seed", GDN_CASES)
def test_gdn_parity(B, L, H, Dh, seg, dtype, dist, h0, dfinal, seed):
    _announce("gdn", B=B, L=L, H=H, Dh=Dh, seg=seg, dtype=dtype, dist=dist, h0=h0, dfinal=dfinal, seed=seed)
    rng = np.random.default_rng(seed)
    ins = _inputs(rng, B, L, H, Dh, dist)
    ts = [to_dev(t, dtype, True) for t in ins]
    h0t = to_dev(rng.standard_normal((B, H, Dh, Dh)) * 0.5, F32, True) if h0 else None
    y, fs = mr.gated_deltanet_scan_with_state(*ts, seg=seg, initial_state=h0t)
    W = _w(rng, (B, L, H, Dh))
    Wf = _w(rng, (B, H, Dh, Dh)) if dfinal else None
    loss = (y * torch.tensor(W, device=y.device)).sum()
    if dfinal:
        loss = loss + (fs * torch.tensor(Wf, device=y.device)).sum()
    loss.backward()
    r = [rounded(t) for t in ts]
    rh0 = rounded(h0t) if h0 else None
    y_o, fs_o = orc.gdn_forward(*r, rh0)
    grads_o = orc.gdn_backward(W, *r, rh0, Wf)
    tol, rep = TOL[dtype], {}
    ftol = TOL[F32] if dtype == F32 else tol
    assert y.dtype == F32 and fs.shape == (B, H, Dh, Dh)
    check("y", y, y_o, ftol, rep)
    check("final", fs, fs_o, ftol, rep)
    for name, t, g in zip(("q", "k", "v", "alpha", "beta"), ts, grads_o):
        assert t.grad.dtype == dtype
        check(f"grad_{name}", t.grad, g, tol, rep)
    if h0:
        check("grad_h0", h0t.grad, grads_o[5], tol, rep)
    print(rep, flush=True)


def test_gdn_exact_recall_full_size():
    """beta_t = 1 and q_t = k_t (unit): k^T S_t = v_t^T exactly in exact
    arithmetic, so y_t = v_t whatever alpha_t and the state before; at the
    bench shape the fp32 kernel keeps it to rounding."""
    B, L, H, Dh = 3, 512, 12, 64
    _announce("gdn_recall", B=B, L=L, H=H, Dh=Dh)
    rng = np.random.default_rng(50)
    k = _unit(rng.standard_normal((B, L, H, Dh)))
    v = rng.standard_normal((B, L, H, Dh))
    alpha = np.exp(-rng.uniform(0.0, 1.0, (B, L, H)))
    kt, vt, at = (to_dev(t, F32) for t in (k, v, alpha))
    bt = torch.ones((B, L, H), dtype=F32, device=kt.device)
    h0 = to_dev(rng.standard_normal((B, H, Dh, Dh)), F32)
    with torch.no_grad():
        y = mr.gated_deltanet_scan(kt, kt, vt, at, bt, initial_state=h0)
    err = (y - vt).abs().max().item() / vt.abs().max().item()
    print({"recall": err}, flush=True)
    assert err < 1e-5


def test_gdn_deterministic():
    """Two runs of forward + backward agree bit for bit (fixed-order sums)."""
    B, L, H, Dh = 2, 256, 6, 64
    _announce("gdn_det", B=B, L=L, H=H, Dh=Dh)
    rng = np.random.default_rng(51)
    ins = _inputs(rng, B, L, H, Dh, "plain")
    W = torch.tensor(_w(rng, (B, L, H, Dh)), device="cuda:0")
    outs = []
    for _ in range(2):
        ts = [to_dev(t, BF16, True) for t in ins]
        y, fs = mr.gated_deltanet_scan_with_state(*ts)
        ((y * W).sum() + fs.sum()).backward()
        outs.append([y.detach(), fs.detach()] + [t.grad for t in ts])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,L,H,dist,h0,seed", [(3, 512, 12, "plain", True, 60), (2, 96, 3, "edges", True, 61),
                                                  (1, 32, 2, "plain", False, 62)])
def test_gdn_chunkwise_forward_matches_sequential(B, L, H, dist, h0, seed):
    """The chunkwise (WY) forward (bf16, Dh 64, T 32, with its workspace)
    against the sequential forward (no workspace) on the same inputs through
    the C ABI: y and every checkpoint, at fp32 accuracy (the chunkwise
    products split fp32 operands into bf16 halves: about 1e-6); both are
    checked against the float64 oracle by the parity cases above."""
    from mlx_recurrence_amd import _lib
    Dh, seg = 64, 32
    _announce("gdn_chunkwise", B=B, L=L, H=H, dist=dist, h0=h0, seed=seed)
    rng = np.random.default_rng(seed)
    q, k, v, a, b = (to_dev(t, BF16) for t in _inputs(rng, B, L, H, Dh, dist))
    h0t = to_dev(rng.standard_normal((B, H, Dh, Dh)) * 0.5, F32) if h0 else None
    nC = L // 32
    ws = _lib.gdn_fwd_workspace(B, L, H, Dh, seg, BF16, q.device)
    assert ws is not None
    res = []
    for w in (None, ws):
        y = torch.full((B, L, H, Dh), float("nan"), dtype=F32, device=q.device)
        ck = torch.full((B, H, nC, Dh, Dh), float("nan"), dtype=F32, device=q.device)
        _lib.gdn_fwd(q, k, v, a, b, h0t, seg, y, ck, w)
        torch.cuda.synchronize()
        res.append((y, ck))
    (ys, cs), (yc, cc) = res
    ey = ((yc - ys).abs().max() / ys.abs().max()).item()
    ec = ((cc - cs).abs().max() / cs.abs().max()).item()
    print({"y": ey, "ckpt": ec}, flush=True)
    assert np.isfinite(ey) and ey < 2e-5 and np.isfinite(ec) and ec < 2e-5


def test_gdn_chunkwise_adjoint_matches_sequential():
    """The chunkwise adjoint pass (bf16, Dh 64, T 32) against the sequential
    one: the same bf16-rounded inputs once as bf16 (chunkwise) and once as
    fp32 (sequential kernels); the fp32 outputs y, the final state and dh0
    (the adjoint carried across every chunk) agree to fp32 accuracy, which
    the 16-bit gradients of the parity cases cannot show."""
    B, L, H, Dh = 2, 256, 4, 64
    _announce("gdn_chunkwise_adjoint", B=B, L=L, H=H, Dh=Dh)
    rng = np.random.default_rng(63)
    ins = [rounded(to_dev(t, BF16)) for t in _inputs(rng, B, L, H, Dh, "edges")]
    h0 = rng.standard_normal((B, H, Dh, Dh)) * 0.5
    W = torch.tensor(_w(rng, (B, L, H, Dh)), device="cuda:0")
    Wf = torch.tensor(_w(rng, (B, H, Dh, Dh)), device="cuda:0")
    res = []
    for dt in (BF16, F32):
        ts = [to_dev(t, dt) for t in ins]
        h0t = to_dev(h0, F32, True)
        y, fs = mr.gated_deltanet_scan_with_state(*ts, initial_state=h0t)
        ((y * W).sum() + (fs * Wf).sum()).backward()
        res.append((y.detach(), fs.detach(), h0t.grad))
    for name, a, b in zip(("y", "final", "dh0"), *res):
        err = ((a - b).abs().max() / b.abs().max()).item()
        print({name: err}, flush=True)
        assert np.isfinite(err) and err < 1e-4, (name, err)


@pytest.mark.parametrize("dist,seed", [("plain", 64), ("edges", 65), ("tiny", 66)])
def test_gdn_chunkwise_gradients_match_sequential(dist, seed):
    """The chunkwise gradient pass (bf16 outputs) against the sequential
    kernels in fp32 on the same bf16-rounded inputs, rounded to bf16: at
    fp32 accuracy of the chunkwise form (about 1e-5) the two roundings
    differ by one bf16 step at most, and only where the exact value lies
    next to a rounding boundary (a small fraction of the elements); an error
    of even 1e-3 would move a large fraction."""
    B, L, H, Dh = 2, 128, 3, 64
    _announce("gdn_chunkwise_grads", B=B, L=L, H=H, Dh=Dh, dist=dist, seed=seed)
    rng = np.random.default_rng(seed)
    ins = [rounded(to_dev(t, BF16)) for t in _inputs(rng, B, L, H, Dh, dist)]
    h0 = rng.standard_normal((B, H, Dh, Dh)) * 0.5
    W = torch.tensor(_w(rng, (B, L, H, Dh)), device="cuda:0")
    Wf = torch.tensor(_w(rng, (B, H, Dh, Dh)), device="cuda:0")
    res = []
    for dt in (BF16, F32):
        ts = [to_dev(t, dt, True) for t in ins]
        h0t = to_dev(h0, F32, True)
        y, fs = mr.gated_deltanet_scan_with_state(*ts, initial_state=h0t)
        ((y * W).sum() + (fs * Wf).sum()).backward()
        res.append([t.grad.float() for t in ts])
    for name, a, b in zip(("dq", "dk", "dv", "dalpha", "dbeta"), *res):
        b16 = b.to(BF16).float()
        step = b16.abs() * 2.0 ** -7 + b16.abs().max() * 1e-5   # one bf16 step (floor near zero)
        diff = (a - b16).abs()
        frac = (diff > 0).float().mean().item()
        worst = (diff / step).max().item()
        print({name: {"moved": frac, "worst_steps": worst}}, flush=True)
        assert worst <= 1.0 and frac < 0.05, (name, frac, worst)
