"""GPU parity of the single-token decode steps (MI355X only).

L consecutive calls of mr.*_step from an initial state must reproduce the
oracle's scan (oracle/recurrence_oracle.py, the reference's per-step
recurrences) over those L tokens: every step's y and the final state.  A
second family continues a chunked prefill: the scan kernels process the first
tokens (*_scan_with_state), the steps continue from the returned final state,
and the concatenated outputs must match the oracle over the whole sequence.
Outputs are fp32 and the arithmetic fp32, so the bar is the fp32 one (1e-5)
whatever the input dtype (the oracle reads the same rounded inputs).
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
BAR = TOL[F32]


def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def _announce(name, **kw):
    print(f"[case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


SSD_CASES = [
    # (B, L, H, Dh, N, dtype, per-head A, seed)
    (2, 24, 3, 64, 16, BF16, True, 0),
    (1, 16, 2, 32, 5, F32, False, 1),       # odd N (scalar state rows), dense A
    (2, 12, 2, 96, 128, F16, True, 2),
    (1, 8, 2, 32, 256, F32, False, 3),      # N = 256: 64 lanes per row
    (8, 3, 80, 64, 128, BF16, True, 4),     # BASELINE config 4's state [8, 80, 64, 128]
    (1, 6, 2, 32, 24, F32, True, 5),        # N = 24: 8 lane groups, the last two past N
    (2, 10, 3, 64, 16, BF16, "1d", 6),      # A_neg [H], as ssd_scan takes it
    (1, 7, 2, 32, 32, F16, "1d", 7),
]


@pytest.mark.parametrize("B,L,H,Dh,N,dtype,per_head,seed", SSD_CASES)
def test_ssd_step(B, L, H, Dh, N, dtype, per_head, seed):
    _announce("ssd_step", B=B, L=L, H=H, Dh=Dh, N=N, dtype=dtype, per_head=per_head)
    rng = np.random.default_rng(seed)
    u = rng.standard_normal((B, L, H, Dh))
    dl = np.abs(rng.standard_normal((B, L, H))) * 0.1 + 0.01
    Bm, Cm = rng.standard_normal((B, L, H, N)), rng.standard_normal((B, L, H, N))
    A = -np.exp(rng.uniform(0, np.log(16), (H, 1 if per_head else N)))
    h0 = rng.standard_normal((B, H, Dh, N)) * 0.5
    ut, dt_, Bt, Ct = (to_dev(v, dtype) for v in (u, dl, Bm, Cm))
    if per_head == "1d":
        At = to_dev(A[:, 0], F32)
    else:
        At = to_dev(A[:, 0], F32)[:, None].expand(H, N) if per_head else to_dev(A, F32)
    state = to_dev(h0, F32).contiguous()
    with torch.no_grad():
        ys = torch.stack([mr.ssd_step(ut[:, t], dt_[:, t], Bt[:, t], Ct[:, t], At, state) for t in range(L)], 1)
    r = [rounded(t) for t in (ut, dt_, Bt, Ct)] + [np.broadcast_to(rounded(At).reshape(H, -1), (H, N))]
    y_o, fs_o = orc.ssd_forward(*r, h0.astype(np.float32).astype(np.float64))
    rep = {}
    check("y", ys, y_o, BAR, rep)
    check("state", state, fs_o, BAR, rep)
    print(rep, flush=True)


def test_ssd_step_keeps_input_dtype(monkeypatch):
    """A bf16 token runs the kernel's bf16 path: the fp32 A_neg does not
    promote u / delta / B / C, so the step launches no cast."""
    from mlx_recurrence_amd import _lib
    seen = []
    real = _lib.ssd_step

    def spy(u, delta, Bm, Cm, A, a_sn, state, y):
        seen.append((u, delta, Bm, Cm, A, a_sn))
        return real(u, delta, Bm, Cm, A, a_sn, state, y)

    monkeypatch.setattr(_lib, "ssd_step", spy)
    dev = torch.device("cuda:0")
    Bsz, H, Dh, N = 2, 3, 64, 16
    u, Bm, Cm = (torch.randn(s_, device=dev).bfloat16() for s_ in ((Bsz, H, Dh), (Bsz, H, N), (Bsz, H, N)))
    d = (torch.rand(Bsz, H, device=dev) * 0.1 + 0.01).bfloat16()
    state = torch.zeros(Bsz, H, Dh, N, device=dev)
    for A in (-torch.rand(H, device=dev) - 0.1, (-torch.rand(H, 1, device=dev) - 0.1).expand(H, N)):
        seen.clear()
        with torch.no_grad():
            mr.ssd_step(u, d, Bm, Cm, A, state)
        (u_, d_, B_, C_, A_, a_sn), = seen
        assert all(t.dtype == torch.bfloat16 for t in (u_, d_, B_, C_))
        assert (u_.data_ptr(), d_.data_ptr(), B_.data_ptr(), C_.data_ptr()) == \
            (u.data_ptr(), d.data_ptr(), Bm.data_ptr(), Cm.data_ptr())
        assert A_.dtype == torch.float32 and A_.shape == (H,) and a_sn == 0


GLA_CASES = [
    # (B, L, H, Dh, dtype, seed)
    (2, 24, 3, 64, BF16, 10),
    (1, 16, 2, 24, F32, 11),     # Dh not a multiple of 4 (scalar rows)
    (1, 12, 2, 128, F16, 12),
    (1, 6, 1, 256, F32, 13),     # Dh = 256: 64 lanes per row
    (1, 8, 2, 20, F32, 14),      # Dh = 20: lane groups past Dh
    (1, 8, 2, 18, BF16, 15),     # Dh = 18: scalar rows, lane groups past Dh
]


@pytest.mark.parametrize("B,L,H,Dh,dtype,seed", GLA_CASES)
def test_gla_step(B, L, H, Dh, dtype, seed):
    _announce("gla_step", B=B, L=L, H=H, Dh=Dh, dtype=dtype)
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((B, L, H, Dh)) / np.sqrt(Dh) for _ in range(3))
    g = _sigmoid(rng.standard_normal((B, L, H)) + 2.0)
    h0 = rng.standard_normal((B, H, Dh, Dh)) * 0.1
    qt, kt, vt, gt = (to_dev(x, dtype) for x in (q, k, v, g))
    state = to_dev(h0, F32).contiguous()
    with torch.no_grad():
        ys = torch.stack([mr.gla_step(qt[:, t], kt[:, t], vt[:, t], gt[:, t], state) for t in range(L)], 1)
    r = [rounded(t) for t in (qt, kt, vt, gt)]
    y_o, fs_o = orc.gla_forward(*r, h0.astype(np.float32).astype(np.float64))
    rep = {}
    check("y", ys, y_o, BAR, rep)
    check("state", state, fs_o, BAR, rep)
    print(rep, flush=True)


@pytest.mark.parametrize("B,L,D,dtype,seed", [(8, 16, 2560, BF16, 20), (2, 20, 100, F32, 21), (3, 9, 96, F16, 22)])
def test_rglru_step(B, L, D, dtype, seed):
    _announce("rglru_step", B=B, L=L, D=D, dtype=dtype)
    rng = np.random.default_rng(seed)
    a = _sigmoid(rng.standard_normal((B, L, D)) + 2.0)
    x = rng.standard_normal((B, L, D))
    h0 = rng.standard_normal((B, D))
    at, xt = to_dev(a, dtype), to_dev(x, dtype)
    state = to_dev(h0, F32).contiguous()
    with torch.no_grad():
        ys = torch.stack([mr.rglru_step(at[:, t], xt[:, t], state) for t in range(L)], 1)
    y_o, fs_o = orc.rglru_forward(rounded(at), rounded(xt), h0.astype(np.float32).astype(np.float64))
    rep = {}
    check("y", ys, y_o, BAR, rep)
    check("state", state, fs_o, BAR, rep)
    print(rep, flush=True)


@pytest.mark.parametrize("B,L,Dp,dtype,seed", [(8, 16, 1280, BF16, 30), (2, 20, 7, F32, 31)])
def test_rotlru_step(B, L, Dp, dtype, seed):
    _announce("rotlru_step", B=B, L=L, Dp=Dp, dtype=dtype)
    rng = np.random.default_rng(seed)
    a = _sigmoid(rng.standard_normal((B, L, Dp)) + 2.0)
    th = rng.uniform(-np.pi, np.pi, (B, L, Dp))
    x = rng.standard_normal((B, L, 2 * Dp))
    h0 = rng.standard_normal((B, 2 * Dp))
    at, ct, st, xt = (to_dev(v, dtype) for v in (a, np.cos(th), np.sin(th), x))
    state = to_dev(h0, F32).contiguous()
    with torch.no_grad():
        ys = torch.stack([mr.rotlru_step(at[:, t], ct[:, t], st[:, t], xt[:, t], state) for t in range(L)], 1)
    r = [rounded(t) for t in (at, ct, st, xt)]
    y_o, fs_o = orc.rotlru_forward(*r, h0.astype(np.float32).astype(np.float64))
    rep = {}
    check("y", ys, y_o, BAR, rep)
    check("state", state, fs_o, BAR, rep)
    print(rep, flush=True)


def test_steps_continue_a_chunked_prefill():
    """Prefill with the scan kernels, then decode with the steps from the
    returned final state: the whole sequence matches the oracle."""
    rng = np.random.default_rng(40)
    B, L0, L1, H, Dh, N = 2, 64, 8, 3, 64, 16
    L = L0 + L1
    u = rng.standard_normal((B, L, H, Dh))
    dl = np.abs(rng.standard_normal((B, L, H))) * 0.1 + 0.01
    Bm, Cm = rng.standard_normal((B, L, H, N)), rng.standard_normal((B, L, H, N))
    A = -np.exp(rng.uniform(0, np.log(16), (H, 1)))
    ut, dt_, Bt, Ct = (to_dev(v, BF16) for v in (u, dl, Bm, Cm))
    At = to_dev(A[:, 0], F32)[:, None].expand(H, N)
    with torch.no_grad():
        y0, state = mr.ssd_scan_with_state(ut[:, :L0], dt_[:, :L0], Bt[:, :L0], Ct[:, :L0], At)
        state = state.contiguous()
        y1 = torch.stack([mr.ssd_step(ut[:, t], dt_[:, t], Bt[:, t], Ct[:, t], At, state) for t in range(L0, L)], 1)
    r = [rounded(t) for t in (ut, dt_, Bt, Ct)] + [np.broadcast_to(rounded(At).reshape(H, -1), (H, N))]
    y_o, fs_o = orc.ssd_forward(*r)
    rep = {}
    check("y", torch.cat([y0, y1], 1), y_o, BAR, rep)
    check("state", state, fs_o, BAR, rep)

    q, k, v = (rng.standard_normal((B, L, H, Dh)) / 8 for _ in range(3))
    g = _sigmoid(rng.standard_normal((B, L, H)) + 2.0)
    qt, kt, vt, gt = (to_dev(x, BF16) for x in (q, k, v, g))
    with torch.no_grad():
        y0, st = mr.gla_scan_with_state(qt[:, :L0], kt[:, :L0], vt[:, :L0], gt[:, :L0])
        st = st.contiguous()
        y1 = torch.stack([mr.gla_step(qt[:, t], kt[:, t], vt[:, t], gt[:, t], st) for t in range(L0, L)], 1)
    y_o, fs_o = orc.gla_forward(*[rounded(t) for t in (qt, kt, vt, gt)])
    check("gla y", torch.cat([y0, y1], 1), y_o, BAR, rep)
    check("gla state", st, fs_o, BAR, rep)
    print(rep, flush=True)


def test_step_rejects_autograd_and_bad_state():
    x = torch.zeros((2, 32), device="cuda:0")
    st = torch.zeros((2, 32), device="cuda:0")
    with pytest.raises(ValueError, match="not differentiable"):
        mr.rglru_step(x.clone().requires_grad_(True), x, st)
    with pytest.raises(ValueError, match="contiguous float32"):
        mr.rglru_step(x, x, st.double())
    with pytest.raises(ValueError, match="state must be"):
        mr.rglru_step(x, x, torch.zeros((2, 16), device="cuda:0"))
