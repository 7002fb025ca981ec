"""Pins the Gated DeltaNet oracle (orc.gdn_forward / gdn_backward) — CPU only.

The reference holds the recurrence as a design (docs/DESIGN_gated_deltanet.md,
no code), so the oracle is pinned against what the mathematics fixes:
  * exact recall (the delta rule's defining property): with beta_t = 1 and a
    unit key, k_t^T S_t = v_t^T whatever alpha_t and the earlier state, so a
    query q_t = k_t reads back v_t exactly;
  * beta = 0: no write and no erase, S_t = (alpha_1 ... alpha_t) S_0, a closed
    form with no recurrence;
  * two steps written out by hand at Dh = 1;
  * backward: central finite differences of every gradient (q, k, v, alpha,
    beta, initial state) and torch float64 autograd of the package's
    per-step torch loop;
  * planted mistakes (erase sign, alpha not on the erase, transposed read-out)
    each fail one of these.
"""
import numpy as np
import pytest
import torch

from oracle import recurrence_oracle as orc
from mlx_recurrence_amd import gated_deltanet_reference

RNG = np.random.default_rng


def _close(a, b, rtol=1e-10, atol=1e-12):
    np.testing.assert_allclose(np.asarray(a), np.asarray(b), rtol=rtol, atol=atol)


def _unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def _inputs(rng, B, L, H, Dh, h0=True):
    q = _unit(rng.standard_normal((B, L, H, Dh)))
    k = _unit(rng.standard_normal((B, L, H, Dh)))
    v = rng.standard_normal((B, L, H, Dh))
    alpha = np.exp(-rng.uniform(0.01, 0.5, (B, L, H)))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, L, H))))
    S0 = rng.standard_normal((B, H, Dh, Dh)) * 0.5 if h0 else None
    return q, k, v, alpha, beta, S0


def _fd_grad(loss, arr, eps=1e-5):
    g = np.empty_like(arr)
    flat, gf = arr.reshape(-1), g.reshape(-1)
    for i in range(flat.size):
        old = flat[i]
        flat[i] = old + eps
        lp = loss()
        flat[i] = old - eps
        lm = loss()
        flat[i] = old
        gf[i] = (lp - lm) / (2 * eps)
    return g


def test_exact_recall_with_unit_write():
    rng = RNG(40)
    q, k, v, alpha, beta, S0 = _inputs(rng, 2, 9, 2, 5)
    beta = np.ones_like(beta)
    y, _ = orc.gdn_forward(k, k, v, alpha, beta, S0)   # query each step with its own key
    _close(y, v, rtol=1e-12, atol=1e-12)


def test_no_write_closed_form():
    rng = RNG(41)
    q, k, v, alpha, beta, S0 = _inputs(rng, 2, 7, 3, 4)
    y, fs = orc.gdn_forward(q, k, v, alpha, np.zeros_like(beta), S0)
    cum = np.cumprod(alpha, axis=1)                                       # [B,L,H]
    want = cum[..., None] * np.einsum("blhi,bhij->blhj", q, S0)
    _close(y, want)
    _close(fs, cum[:, -1, :, None, None] * S0)


def test_two_steps_by_hand():
    # Dh = 1: S_t = a_t (1 - b_t k_t^2) S_{t-1} + b_t k_t v_t,  o_t = q_t S_t
    q = np.array([0.7, -1.2]).reshape(1, 2, 1, 1)
    k = np.array([0.9, 0.4]).reshape(1, 2, 1, 1)
    v = np.array([1.5, -0.3]).reshape(1, 2, 1, 1)
    a = np.array([0.8, 0.6]).reshape(1, 2, 1)
    b = np.array([0.5, 0.25]).reshape(1, 2, 1)
    S0 = np.array([2.0]).reshape(1, 1, 1, 1)
    S1 = 0.8 * (1 - 0.5 * 0.81) * 2.0 + 0.5 * 0.9 * 1.5
    S2 = 0.6 * (1 - 0.25 * 0.16) * S1 + 0.25 * 0.4 * -0.3
    y, fs = orc.gdn_forward(q, k, v, a, b, S0)
    _close(y.ravel(), [0.7 * S1, -1.2 * S2])
    _close(fs.ravel(), [S2])


def test_backward_finite_differences():
    rng = RNG(42)
    q, k, v, alpha, beta, S0 = _inputs(rng, 1, 5, 2, 3)
    W = rng.standard_normal(q.shape)
    Wf = rng.standard_normal(S0.shape)
    args = [q, k, v, alpha, beta, S0]

    def loss():
        y, fs = orc.gdn_forward(*args)
        return float((y * W).sum() + (fs * Wf).sum())

    grads = orc.gdn_backward(W, *args, dfinal=Wf)
    for name, arr, g in zip(("q", "k", "v", "alpha", "beta", "h0"), args, grads):
        np.testing.assert_allclose(g, _fd_grad(loss, arr), rtol=1e-6, atol=1e-8, err_msg=name)


def test_backward_matches_torch_autograd_of_reference_loop():
    rng = RNG(43)
    q, k, v, alpha, beta, S0 = _inputs(rng, 2, 20, 2, 4)
    W = rng.standard_normal(q.shape)
    ts = [torch.tensor(a, requires_grad=True) for a in (q, k, v, alpha, beta, S0)]
    y = gated_deltanet_reference(*ts[:5], initial_state=ts[5])
    (y * torch.tensor(W)).sum().backward()
    y_o, _ = orc.gdn_forward(q, k, v, alpha, beta, S0)
    _close(y.detach().numpy(), y_o, rtol=1e-12, atol=1e-13)
    for name, t, g in zip(("q", "k", "v", "alpha", "beta", "h0"), ts, orc.gdn_backward(W, q, k, v, alpha, beta, S0)):
        np.testing.assert_allclose(t.grad.numpy(), g, rtol=1e-9, atol=1e-11, err_msg=name)


@pytest.mark.parametrize("plant", ["erase_sign", "alpha_off_erase", "transposed_readout"])
def test_checks_catch_planted_mistakes(plant):
    """Restatements with a planted mistake fail the exact-recall check."""
    rng = RNG(44)
    q, k, v, alpha, beta, S0 = _inputs(rng, 1, 6, 1, 4)
    beta = np.ones_like(beta)
    S = S0.copy()
    ys = []
    for t in range(k.shape[1]):
        kt, vt, a, b = k[:, t], v[:, t], alpha[:, t, :, None, None], beta[:, t, :, None, None]
        p = np.einsum("bhi,bhij->bhj", kt, S)
        kp = kt[..., :, None] * p[..., None, :]
        kv = kt[..., :, None] * vt[..., None, :]
        if plant == "erase_sign":
            S = a * (S + b * kp) + b * kv
        elif plant == "alpha_off_erase":
            S = a * S - b * kp + b * kv
        else:
            S = a * (S - b * kp) + b * kv
        read = np.einsum("bhij,bhj->bhi", S, kt) if plant == "transposed_readout" else np.einsum("bhi,bhij->bhj", kt, S)
        ys.append(read)
    y_bad = np.stack(ys, 1)
    assert not np.allclose(y_bad, v, atol=1e-6)
    y, _ = orc.gdn_forward(k, k, v, alpha, beta, S0)
    _close(y, v, rtol=1e-12, atol=1e-12)
