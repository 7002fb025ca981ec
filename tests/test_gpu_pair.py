"""The SSD backward in pair mode (MI355X only): many heads with a wide state
(N >= 64, Dh <= 64, B*H >= 320, an even chunk count) run the per-head adjoint
scan storing the adjoint leaving every second chunk only, and one workgroup
per pair of chunks that carries the adjoint across the pair itself.

Shapes: B=4 L=128 H=80 Dh=64 N=128 bf16 (320 heads, 4 chunks per head: two
pairs), the smallest that takes the mode with more than one pair per head;
the guard test also at L=64 (one pair per head).
  - Through the C ABI, with guard regions after the workspace (as large as the
    workspace itself) and after every output, filled with a byte pattern:
    nothing may be written past the sizes the library states
    (rr_ssd_workspace_bytes, the output shapes).
  - Through the C ABI: all batch rows of heads 0, 37 and 79 against the
    float64 oracle (oracle/recurrence_oracle.py, reference ssd.py:203-268),
    so dA of those heads is complete, compared per state n (dA_neg [H, N] as
    the kernels form it; the sum over n of one head can cancel to a value two
    orders below its terms); bars as in the other parity tests (fp32 outputs
    1e-5, bf16 gradients 2e-2).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from mlx_recurrence_amd import _lib
from oracle import recurrence_oracle as orc
from tests.gpu_util import rel_err

import mlx_recurrence_amd as mr

pytestmark = pytest.mark.gpu

B, L, H, Dh, N, SEG = 4, 128, 80, 64, 128, 32
HEADS = (0, 37, 79)
PATTERN = 0x5A
GUARD_OUT = 4096   # bytes past each output


def _inputs(seed, L=L):
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    u = torch.randn((B, L, H, Dh), generator=g, device=dev).to(bf)
    delta = (torch.randn((B, L, H), generator=g, device=dev).abs() * 0.1 + 0.01).to(bf)
    Bm = torch.randn((B, L, H, N), generator=g, device=dev).to(bf)
    Cm = torch.randn((B, L, H, N), generator=g, device=dev).to(bf)
    A = -torch.exp(torch.rand((H,), generator=g, device=dev) * math.log(16.0))
    W = torch.randn((B, L, H, Dh), generator=g, device=dev)
    return u, delta, Bm, Cm, A, W


def _a64(n):
    return (n + 63) // 64 * 64


def _assert_pair_mode(Bsz, seq, Hh, dh, n_st):
    """The backward workspace the library asks for at this shape is the pair
    mode's (per-chunk decays, dA partials and one adjoint per pair of chunks,
    each part 256-byte aligned), which tells the mode apart from the
    per-chunk pipelined one (an adjoint per chunk) and the direct one."""
    nC = seq // 32
    want = 4 * (_a64(Bsz * Hh * nC) + _a64(Bsz * Hh * (nC // 2) * n_st) + _a64(Bsz * Hh * (nC // 2) * dh * n_st))
    got = _lib.load().rr_ssd_workspace_bytes(Bsz, seq, Hh, dh, n_st, SEG, 0, _lib.DTYPE_CODE[torch.bfloat16], 1)
    assert got == want, f"not the pair mode at B={Bsz} L={seq} H={Hh} Dh={dh} N={n_st}: {got} != {want}"


def _guarded(shape, dtype, guard_bytes):
    """An output tensor of `shape` that is the prefix of a larger buffer whose
    tail (guard_bytes) holds PATTERN; returns (tensor, guard bytes view)."""
    n = int(np.prod(shape)) * torch.tensor([], dtype=dtype).element_size()
    buf = torch.full((n + guard_bytes,), PATTERN, dtype=torch.uint8, device="cuda:0")
    return buf[:n].view(dtype).view(shape), buf[n:]


@pytest.mark.parametrize("L", [L, 64], ids=["two_pairs", "one_pair"])
def test_pair_mode_writes_inside_its_buffers(L):
    print(f"[case] ssd pair-mode guards B={B} L={L} H={H} Dh={Dh} N={N} bf16", flush=True)
    _assert_pair_mode(B, L, H, Dh, N)
    u, delta, Bm, Cm, A, dy = _inputs(11, L)
    nC = L // _lib.chunk_len(L, SEG)
    y = torch.empty((B, L, H, Dh), dtype=torch.float32, device=u.device)
    ckpt = torch.empty((B, H, nC, Dh, N), dtype=torch.float32, device=u.device)
    wsf = _lib.ssd_workspace(B, L, H, Dh, N, SEG, 0, u.dtype, 0, u.device)
    _lib.ssd_fwd(u, delta, Bm, Cm, A, 0, None, SEG, y, ckpt, wsf)
    nws = _lib.load().rr_ssd_workspace_bytes(B, L, H, Dh, N, SEG, 0, _lib.DTYPE_CODE[u.dtype], 1)
    assert nws > 0
    ws_buf = torch.full((2 * nws,), PATTERN, dtype=torch.uint8, device=u.device)
    ws, ws_guard = ws_buf[:nws], ws_buf[nws:]
    outs = [_guarded(u.shape, u.dtype, GUARD_OUT), _guarded(delta.shape, delta.dtype, GUARD_OUT),
            _guarded(Bm.shape, Bm.dtype, GUARD_OUT), _guarded(Cm.shape, Cm.dtype, GUARD_OUT),
            _guarded((H, N), torch.float32, GUARD_OUT)]   # dA_neg [H, N] at the C ABI
    _lib.ssd_bwd(dy, None, u, delta, Bm, Cm, A, 0, None, ckpt, SEG, *(o for o, _ in outs), None, ws)
    torch.cuda.synchronize()
    assert bool((ws_guard == PATTERN).all()), "the backward wrote past its workspace"
    for name, (o, gd) in zip(("du", "ddelta", "dB", "dC", "dA"), outs):
        assert bool((gd == PATTERN).all()), f"the backward wrote past {name}"
        assert bool(torch.isfinite(o.float()).all()), f"{name} not finite"


@pytest.fixture(scope="module")
def pair_run():
    """Forward + backward through the C ABI (so dA_neg comes per state n,
    [H, N], as the kernels form it); returns float64 CPU slices of the
    selected heads."""
    print(f"[case] ssd pair-mode parity B={B} L={L} H={H} Dh={Dh} N={N} bf16", flush=True)
    _assert_pair_mode(B, L, H, Dh, N)
    u, delta, Bm, Cm, A, W = _inputs(12)
    nC = L // _lib.chunk_len(L, SEG)
    y = torch.empty((B, L, H, Dh), dtype=torch.float32, device=u.device)
    ckpt = torch.empty((B, H, nC, Dh, N), dtype=torch.float32, device=u.device)
    _lib.ssd_fwd(u, delta, Bm, Cm, A, 0, None, SEG, y, ckpt,
                 _lib.ssd_workspace(B, L, H, Dh, N, SEG, 0, u.dtype, 0, u.device))
    grads = [torch.empty_like(u), torch.empty_like(delta), torch.empty_like(Bm), torch.empty_like(Cm),
             torch.empty((H, N), dtype=torch.float32, device=u.device)]
    _lib.ssd_bwd(W, None, u, delta, Bm, Cm, A, 0, None, ckpt, SEG, *grads, None,
                 _lib.ssd_workspace(B, L, H, Dh, N, SEG, 0, u.dtype, 1, u.device))
    torch.cuda.synchronize()
    idx = torch.tensor(HEADS, device=u.device)

    def cpu(t, axis):
        return t.detach().index_select(axis, idx).double().cpu().numpy()

    return dict(u=cpu(u, 2), delta=cpu(delta, 2), Bm=cpu(Bm, 2), Cm=cpu(Cm, 2), A=cpu(A, 0), W=cpu(W, 2),
                y=cpu(y, 2), fs=cpu(ckpt[:, :, nC - 1], 1), du=cpu(grads[0], 2), dd=cpu(grads[1], 2),
                dB=cpu(grads[2], 2), dC=cpu(grads[3], 2), dA=cpu(grads[4], 0))


@pytest.mark.parametrize("j", range(len(HEADS)), ids=[f"head{h}" for h in HEADS])
def test_pair_mode_parity(pair_run, j):
    r = pair_run
    sl = (slice(None), slice(None), slice(j, j + 1))
    u, dl, Bm, Cm = r["u"][sl], r["delta"][:, :, j:j + 1], r["Bm"][sl], r["Cm"][sl]
    A = np.repeat(r["A"][j:j + 1, None], N, axis=1)
    y_o, fs_o = orc.ssd_forward(u, dl, Bm, Cm, A)
    du_o, dd_o, dB_o, dC_o, dA_o, _ = orc.ssd_backward(r["W"][sl], u, dl, Bm, Cm, A)
    errs = {
        "y": rel_err(r["y"][sl], y_o), "final": rel_err(r["fs"][:, j:j + 1], fs_o),
        "grad_A": rel_err(r["dA"][j:j + 1], dA_o),   # per state n: [1, N]
        "grad_u": rel_err(r["du"][sl], du_o), "grad_delta": rel_err(r["dd"][:, :, j:j + 1], dd_o),
        "grad_B": rel_err(r["dB"][sl], dB_o), "grad_C": rel_err(r["dC"][sl], dC_o),
    }
    print(f"ssd pair head {HEADS[j]}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k in ("y", "final", "grad_A"):
        assert errs[k] < 1e-5, (k, errs)
    for k in ("grad_u", "grad_delta", "grad_B", "grad_C"):
        assert errs[k] < 2e-2, (k, errs)


def test_pair_mode_initial_state_and_final_cotangent():
    """N = 64, three pairs per head (L = 192: more than the four chunks of the
    direct mode), with an initial state and a loss on the final state: the
    entering state of the first chunk, the final-state cotangent through the
    adjoint scan and dh0 (through the public API; heads 0 and 79 against
    the oracle)."""
    n_st, seq = 64, 192
    print(f"[case] ssd pair-mode h0 + dfinal B={B} L={seq} H={H} Dh={Dh} N={n_st} bf16", flush=True)
    _assert_pair_mode(B, seq, H, Dh, n_st)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(13)
    bf = torch.bfloat16
    u = torch.randn((B, seq, H, Dh), generator=g, device=dev).to(bf)
    delta = (torch.randn((B, seq, H), generator=g, device=dev).abs() * 0.1 + 0.01).to(bf)
    Bm = torch.randn((B, seq, H, n_st), generator=g, device=dev).to(bf)
    Cm = torch.randn((B, seq, H, n_st), generator=g, device=dev).to(bf)
    A = -torch.exp(torch.rand((H,), generator=g, device=dev) * math.log(16.0))
    h0 = torch.randn((B, H, Dh, n_st), generator=g, device=dev)
    W = torch.randn((B, seq, H, Dh), generator=g, device=dev)
    V = torch.randn((B, H, Dh, n_st), generator=g, device=dev)
    xs = [t.requires_grad_(True) for t in (u, delta, Bm, Cm, A, h0)]
    y, fs = mr.ssd_scan_with_state(xs[0], xs[1], xs[2], xs[3], xs[4], seg=SEG, initial_state=xs[5])
    ((y * W).sum() + (fs * V).sum()).backward()
    torch.cuda.synchronize()
    for h in (0, 79):
        def sel(t, axis):
            return t.detach().select(axis, h).unsqueeze(axis).double().cpu().numpy()
        ui, di, bi, ci = sel(u, 2), sel(delta, 2), sel(Bm, 2), sel(Cm, 2)
        Ai = np.repeat(A.detach()[h].double().cpu().numpy().reshape(1, 1), n_st, axis=1)
        h0i, Vi, Wi = sel(h0, 1), sel(V, 1), sel(W, 2)
        y_o, fs_o = orc.ssd_forward(ui, di, bi, ci, Ai, h0=h0i)
        du_o, dd_o, dB_o, dC_o, dA_o, dh0_o = orc.ssd_backward(Wi, ui, di, bi, ci, Ai, h0=h0i, dfinal=Vi)
        errs = {
            "y": rel_err(sel(y, 2), y_o), "final": rel_err(sel(fs, 1), fs_o),
            "grad_h0": rel_err(sel(xs[5].grad, 1), dh0_o),
            "grad_u": rel_err(sel(xs[0].grad, 2), du_o), "grad_delta": rel_err(sel(xs[1].grad, 2), dd_o),
            "grad_B": rel_err(sel(xs[2].grad, 2), dB_o), "grad_C": rel_err(sel(xs[3].grad, 2), dC_o),
        }
        print(f"ssd pair h0/dfinal head {h}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
        for k in ("y", "final", "grad_h0"):
            assert errs[k] < 1e-5, (h, k, errs)
        for k in ("grad_u", "grad_delta", "grad_B", "grad_C"):
            assert errs[k] < 2e-2, (h, k, errs)
