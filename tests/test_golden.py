"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored vector (a change to the oracle
shows up here).  GPU: the kernels, through the public API, match the stored
outputs and gradients of each fixture (fp32 inputs, normalised error < 1e-5)."""
import pathlib

import numpy as np
import pytest
import torch

from oracle import recurrence_oracle as orc
from tests.gpu_util import rel_err

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _same(got, want):
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-14)


def test_oracle_reproduces_fixtures():
    for name in ("ssd_c0", "ssd_ref_shape"):
        f = _load(name)
        ins = (f["u"], f["delta"], f["B"], f["C"], f["A_neg"])
        y, fs = orc.ssd_forward(*ins)
        _same(y, f["y"])
        _same(fs, f["final"])
        for g, k in zip(orc.ssd_backward(f["dy"], *ins)[:5], ("du", "ddelta", "dB", "dC", "dA_neg")):
            _same(g, f[k])
    f = _load("gla_small")
    ins = (f["q"], f["k"], f["v"], f["gates"])
    _same(orc.gla_forward(*ins)[0], f["y"])
    for g, k in zip(orc.gla_backward(f["dy"], *ins)[:4], ("dq", "dk", "dv", "dgates")):
        _same(g, f[k])
    f = _load("rglru_small")
    _same(orc.rglru_forward(f["a"], f["x"])[0], f["y"])
    for g, k in zip(orc.rglru_backward(f["dy"], f["a"], f["x"])[:2], ("da", "dx")):
        _same(g, f[k])
    f = _load("rotlru_small")
    ins = (f["a"], f["cs"], f["sn"], f["x"])
    _same(orc.rotlru_forward(*ins)[0], f["y"])
    for g, k in zip(orc.rotlru_backward(f["dy"], *ins)[:4], ("da", "dcs", "dsn", "dx")):
        _same(g, f[k])


def _run(fn, names, f, out_names):
    dev = torch.device("cuda:0")
    xs = [torch.tensor(f[n], dtype=torch.float32, device=dev, requires_grad=True) for n in names]
    y, fs = fn(*xs)
    (y * torch.tensor(f["dy"], dtype=torch.float32, device=dev)).sum().backward()
    errs = {"y": rel_err(y, f["y"]), "final": rel_err(fs, f["final"])}
    errs.update({k: rel_err(x.grad, f[k]) for x, k in zip(xs, out_names)})
    assert max(errs.values()) < 1e-5, errs


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["ssd_c0", "ssd_ref_shape"])
def test_gpu_ssd_fixture(name):
    import mlx_recurrence_amd as mr
    _run(mr.ssd_scan_with_state, ("u", "delta", "B", "C", "A_neg"), _load(name),
         ("du", "ddelta", "dB", "dC", "dA_neg"))


@pytest.mark.gpu
def test_gpu_gla_fixture():
    import mlx_recurrence_amd as mr
    _run(mr.gla_scan_with_state, ("q", "k", "v", "gates"), _load("gla_small"), ("dq", "dk", "dv", "dgates"))


@pytest.mark.gpu
def test_gpu_rglru_fixture():
    import mlx_recurrence_amd as mr
    _run(mr.rglru_scan_with_state, ("a", "x"), _load("rglru_small"), ("da", "dx"))


@pytest.mark.gpu
def test_gpu_rotlru_fixture():
    import mlx_recurrence_amd as mr
    _run(mr.rotlru_scan_with_state, ("a", "cs", "sn", "x"), _load("rotlru_small"), ("da", "dcs", "dsn", "dx"))
