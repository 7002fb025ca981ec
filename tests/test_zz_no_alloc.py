"""rr_ssd_bwd_noalloc (the SSD backward on the library's static device scratch,
for callers that cannot allocate) against rr_ssd_bwd with a caller workspace,
through the C ABI on the same inputs: bit-identical gradients, on consecutive
calls whose second and third inputs are smaller than the first (the scratch
keeps the previous call's contents)."""
from __future__ import annotations

import math

import pytest
import torch

from mlx_recurrence_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(B, L, H, Dh, N, dense_A, dtype, seed):
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    u = torch.randn((B, L, H, Dh), generator=g, device=dev).to(dtype)
    delta = (torch.randn((B, L, H), generator=g, device=dev).abs() * 0.1 + 0.01).to(dtype)
    Bm = torch.randn((B, L, H, N), generator=g, device=dev).to(dtype)
    Cm = torch.randn((B, L, H, N), generator=g, device=dev).to(dtype)
    if dense_A:
        A = -torch.exp(torch.rand((H, N), generator=g, device=dev) * math.log(16.0))
    else:
        A = -torch.exp(torch.rand((H,), generator=g, device=dev) * math.log(16.0))
    dy = torch.randn((B, L, H, Dh), generator=g, device=dev)
    return u, delta, Bm, Cm, A, dy


def _grads(u, delta, Bm, Cm):
    B, L, H, Dh = u.shape
    N = Bm.shape[-1]
    return [torch.empty_like(u), torch.empty_like(delta), torch.empty_like(Bm), torch.empty_like(Cm),
            torch.empty((H, N), dtype=torch.float32, device=u.device)]


CALLS = [
    # (B, L, H, Dh, N, dense A, dtype, seed): BASELINE config 1, then smaller calls
    (3, 512, 12, 64, 16, False, torch.bfloat16, 1),
    (1, 256, 4, 64, 16, False, torch.bfloat16, 2),
    (1, 64, 2, 32, 8, True, torch.float32, 3),     # dense A, fp32: the VALU engine
]


def test_noalloc_matches_workspace_entry_point():
    for (B, L, H, Dh, N, dense, dtype, seed) in CALLS:
        print(f"[case] ssd_bwd_noalloc B={B} L={L} H={H} Dh={Dh} N={N} dense_A={dense} {dtype}", flush=True)
        u, delta, Bm, Cm, A, dy = _inputs(B, L, H, Dh, N, dense, dtype, seed)
        a_sn = 1 if dense else 0
        nC = L // _lib.chunk_len(L, 32)
        y = torch.empty((B, L, H, Dh), dtype=torch.float32, device=u.device)
        ckpt = torch.empty((B, H, nC, Dh, N), dtype=torch.float32, device=u.device)
        wsf = _lib.ssd_workspace(B, L, H, Dh, N, 32, a_sn, dtype, 0, u.device)
        _lib.ssd_fwd(u, delta, Bm, Cm, A, a_sn, None, 32, y, ckpt, wsf)
        want = _grads(u, delta, Bm, Cm)
        wsb = _lib.ssd_workspace(B, L, H, Dh, N, 32, a_sn, dtype, 1, u.device)
        _lib.ssd_bwd(dy, None, u, delta, Bm, Cm, A, a_sn, None, ckpt, 32, *want, None, wsb)
        got = _grads(u, delta, Bm, Cm)
        for t in got:                       # no stale values can pass for results
            t.view(torch.uint8).fill_(0xFF)
        _lib.ssd_bwd_noalloc(dy, None, u, delta, Bm, Cm, A, a_sn, None, ckpt, 32, *got, None)
        torch.cuda.synchronize()
        for name, w, g in zip(("du", "ddelta", "dB", "dC", "dA"), want, got):
            assert torch.equal(w.view(torch.uint8), g.view(torch.uint8)), f"{name} differs (B={B} L={L} H={H})"
