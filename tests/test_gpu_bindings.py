"""The C++ autograd bindings (mlx_recurrence_amd._autograd) against the Python
torch.autograd.Functions of ssd.py / gla.py (MI355X only): both drive the same
kernels through the same C ABI, so outputs and every gradient must agree bit
for bit, with and without an initial state and a final-state cotangent, and
for A_neg given as [H], as a broadcast [H, N] and dense.  The 1-D A_neg's
gradient is the per-head sum of the broadcast form's."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_recurrence_amd as mr
from mlx_recurrence_amd import _lib
from mlx_recurrence_amd.gla import _GLAScan
from mlx_recurrence_amd.ssd import _SSDScan

pytestmark = pytest.mark.gpu


def _leaves(ts):
    return [t.detach().clone().requires_grad_(True) if t is not None else None for t in ts]


def _run_both(fn_ext, fn_py, inputs, seg, w_y, w_f):
    outs = []
    for fn in (fn_ext, fn_py):
        xs = _leaves(inputs)
        y, fs = fn(xs, seg)
        loss = (y * w_y).sum() + ((fs * w_f).sum() if w_f is not None else 0.0)
        loss.backward()
        outs.append([y.detach(), fs.detach()] + [x.grad for x in xs if x is not None])
    return outs


@pytest.mark.parametrize("a_form", ["heads", "broadcast", "dense"])
@pytest.mark.parametrize("h0,dfinal", [(False, False), (True, True)])
def test_ssd_bindings_agree(a_form, h0, dfinal):
    ext = _lib.autograd_ext()
    assert ext is not None, "the C++ autograd bindings are not built"
    print(f"[case] ssd bindings a_form={a_form} h0={h0} dfinal={dfinal}", flush=True)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(7)
    B, L, H, Dh, N = 2, 256, 3, 64, 16
    u = torch.randn(B, L, H, Dh, generator=g).bfloat16().to(dev)
    d = (torch.rand(B, L, H, generator=g) * 0.1 + 0.01).bfloat16().to(dev)
    Bm = torch.randn(B, L, H, N, generator=g).bfloat16().to(dev)
    Cm = torch.randn(B, L, H, N, generator=g).bfloat16().to(dev)
    A = (-torch.rand(H, N if a_form == "dense" else 1, generator=g) - 0.5).to(dev)
    A = A[:, 0] if a_form == "heads" else (A.expand(H, N) if a_form == "broadcast" else A)
    S0 = torch.randn(B, H, Dh, N, generator=g).to(dev) * 0.1 if h0 else None
    w_y = torch.randn(B, L, H, Dh, generator=g).to(dev)
    w_f = torch.randn(B, H, Dh, N, generator=g).to(dev) if dfinal else None

    def via_ext(xs, seg):
        return ext.ssd_scan(*xs, seg)

    def via_py(xs, seg):
        return _SSDScan.apply(*xs, seg)

    a_ext, a_py = _run_both(via_ext, via_py, [u, d, Bm, Cm, A, S0], 32, w_y, w_f)
    for i, (x, y_) in enumerate(zip(a_ext, a_py)):
        assert x.shape == y_.shape and x.dtype == y_.dtype, i
        assert torch.equal(x, y_), f"output {i} differs"
    if a_form == "heads":   # the public API with [H] against the broadcast form
        xs = _leaves([u, d, Bm, Cm])
        A1 = A.detach().clone().requires_grad_(True)
        A2 = A.detach().clone().requires_grad_(True)
        (mr.ssd_scan(*xs, A1) * w_y).sum().backward()
        (mr.ssd_scan(*xs, A2[:, None].expand(H, N)) * w_y).sum().backward()
        np.testing.assert_allclose(A1.grad.cpu().numpy(), A2.grad.cpu().numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("h0,dfinal", [(False, False), (True, True)])
def test_gla_bindings_agree(h0, dfinal):
    ext = _lib.autograd_ext()
    assert ext is not None, "the C++ autograd bindings are not built"
    print(f"[case] gla bindings h0={h0} dfinal={dfinal}", flush=True)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(8)
    B, L, H, Dh = 2, 256, 3, 64
    q, k, v = ((torch.randn(B, L, H, Dh, generator=g) / 8).bfloat16().to(dev) for _ in range(3))
    gates = torch.sigmoid(torch.randn(B, L, H, generator=g) + 2).bfloat16().to(dev)
    S0 = torch.randn(B, H, Dh, Dh, generator=g).to(dev) * 0.1 if h0 else None
    w_y = torch.randn(B, L, H, Dh, generator=g).to(dev)
    w_f = torch.randn(B, H, Dh, Dh, generator=g).to(dev) if dfinal else None

    def via_ext(xs, seg):
        return ext.gla_scan(*xs, seg)

    def via_py(xs, seg):
        return _GLAScan.apply(*xs, seg)

    a_ext, a_py = _run_both(via_ext, via_py, [q, k, v, gates, S0], 32, w_y, w_f)
    for i, (x, y_) in enumerate(zip(a_ext, a_py)):
        assert x.shape == y_.shape and x.dtype == y_.dtype, i
        assert torch.equal(x, y_), f"output {i} differs"
