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


@pytest.mark.parametrize("kind", ["ssd", "gla"])
def test_bindings_release_workspace_and_checkpoints(kind):
    """The C++ bindings' allocations end with their use: after backward, with
    the gradients and y alive, the device holds the gradients, y and the
    inputs only (the backward's workspace is released when the pass returns,
    and the checkpoints with the autograd graph); y alone does not hold the
    checkpoints."""
    ext = _lib.autograd_ext()
    assert ext is not None, "the C++ autograd bindings are not built"
    print(f"[case] bindings memory {kind}", flush=True)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(9)
    # more than 16 chunks: the pipelined backward, whose workspace holds every chunk's adjoint
    B, L, H, Dh, N = 1, 1024, 3, 64, 16
    if kind == "ssd":
        xs = [torch.randn(B, L, H, Dh, generator=g), torch.rand(B, L, H, generator=g) * 0.1 + 0.01,
              torch.randn(B, L, H, N, generator=g), torch.randn(B, L, H, N, generator=g)]
        xs = [x.bfloat16().to(dev).requires_grad_(True) for x in xs]
        A = (-torch.rand(H, generator=g) - 0.5).to(dev).requires_grad_(True)
        ws = _lib.ssd_workspace(B, L, H, Dh, N, 32, 0, torch.bfloat16, 1, dev)
        ck_bytes = B * H * (L // 32) * Dh * N * 4
        xs.append(A)

        def call(ys):
            return ext.ssd_scan(*ys, None, 32)
    else:
        xs = [(torch.randn(B, L, H, Dh, generator=g) / 8).bfloat16().to(dev).requires_grad_(True) for _ in range(3)]
        xs.append(torch.sigmoid(torch.randn(B, L, H, generator=g) + 2).bfloat16().to(dev).requires_grad_(True))
        ws = _lib.gla_workspace(B, L, H, Dh, 32, torch.bfloat16, 1, dev)
        ck_bytes = B * H * (L // 32) * Dh * Dh * 4

        def call(ys):
            return ext.gla_scan(*ys, None, 32)
    ws_bytes = 0 if ws is None else ws.numel()
    del ws
    assert ws_bytes > 256 * 1024, "the case is meant to have a sizeable backward workspace"
    w_y = torch.randn(B, L, H, Dh, generator=g).to(dev)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    y, fs = call(xs)
    del fs
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated(dev) - base
    y_bytes = y.numel() * 4
    # forward: y and the checkpoints (saved by the graph), no workspace
    assert held <= y_bytes + ck_bytes + 64 * 1024, (held, y_bytes, ck_bytes)
    (y * w_y).sum().backward()
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated(dev) - base
    grad_bytes = sum(x.grad.numel() * x.grad.element_size() for x in xs)
    # graph freed: y and the gradients remain (256-byte piece alignment, allocator rounding)
    assert held <= y_bytes + grad_bytes + 64 * 1024, (held, y_bytes, grad_bytes, ws_bytes)
    assert held < y_bytes + grad_bytes + ws_bytes // 2
