"""Generate the golden fixtures tests/golden/*.npz from the float64 oracle.

The reference (D-CSIL/mlx-recurrence) holds no stored vectors: its tests draw
mx.random inputs at run time and compare against its own per-step loop.  These
fixtures are therefore produced by the pinned oracle (oracle/recurrence_oracle.py,
checked by tests/test_oracle.py) on seeded inputs with the reference tests'
distributions and BASELINE config 0's shape, so that GPU runs compare against
fixed numbers and any later change of the oracle shows up as a diff.

Inputs are rounded to float32 before the oracle sees them (the GPU tests feed
the same float32 values).  Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import recurrence_oracle as orc  # noqa: E402


def f32(a):
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def ssd_c0():
    """B1 L128 H2 Dh32 N16, A per head broadcast over N."""
    rng = np.random.default_rng(100)
    B, L, H, Dh, N = 1, 128, 2, 32, 16
    u = f32(rng.standard_normal((B, L, H, Dh)))
    delta = f32(np.abs(rng.standard_normal((B, L, H))) * 0.1 + 0.01)
    Bm = f32(rng.standard_normal((B, L, H, N)))
    Cm = f32(rng.standard_normal((B, L, H, N)))
    A = f32(np.repeat(-np.exp(rng.uniform(0, np.log(16), (H, 1))), N, axis=1))
    dy = f32(rng.standard_normal((B, L, H, Dh)))
    y, fs = orc.ssd_forward(u, delta, Bm, Cm, A)
    du, dd, dB, dC, dA, _ = orc.ssd_backward(dy, u, delta, Bm, Cm, A)
    return dict(u=u, delta=delta, B=Bm, C=Cm, A_neg=A, dy=dy, y=y, final=fs,
                du=du, ddelta=dd, dB=dB, dC=dC, dA_neg=dA)


def ssd_ref_shape():
    """test_v2_ssd.py:26-30 shape (2, 64, 2, 64, 8, seg=32), its distributions."""
    rng = np.random.default_rng(101)
    B, L, H, Dh, N = 2, 64, 2, 64, 8
    u = f32(rng.standard_normal((B, L, H, Dh)) * 0.5)
    delta = f32(np.abs(rng.standard_normal((B, L, H))) * 0.05 + 0.001)
    Bm = f32(rng.standard_normal((B, L, H, N)) * 0.5)
    Cm = f32(rng.standard_normal((B, L, H, N)) * 0.5)
    A = f32(-np.abs(rng.standard_normal((H, N))) - 0.1)
    dy = f32(rng.standard_normal((B, L, H, Dh)))
    y, fs = orc.ssd_forward(u, delta, Bm, Cm, A)
    du, dd, dB, dC, dA, _ = orc.ssd_backward(dy, u, delta, Bm, Cm, A)
    return dict(u=u, delta=delta, B=Bm, C=Cm, A_neg=A, dy=dy, y=y, final=fs,
                du=du, ddelta=dd, dB=dB, dC=dC, dA_neg=dA)


def gla_small():
    """test_v2_gla.py:11-18 distributions, shape (1, 64, 2, 32)."""
    rng = np.random.default_rng(102)
    B, L, H, Dh = 1, 64, 2, 32
    q = f32(rng.standard_normal((B, L, H, Dh)) * Dh ** -0.5)
    k = f32(rng.standard_normal((B, L, H, Dh)) * 0.5)
    v = f32(rng.standard_normal((B, L, H, Dh)) * 0.5)
    g = f32(1 / (1 + np.exp(-(rng.standard_normal((B, L, H)) + 2))))
    dy = f32(rng.standard_normal((B, L, H, Dh)))
    y, fs = orc.gla_forward(q, k, v, g)
    dq, dk, dv, dg, _ = orc.gla_backward(dy, q, k, v, g)
    return dict(q=q, k=k, v=v, gates=g, dy=dy, y=y, final=fs, dq=dq, dk=dk, dv=dv, dgates=dg)


def rglru_small():
    """test_v2_rglru.py:199-219: negative gates, shape (2, 64, 64)."""
    rng = np.random.default_rng(103)
    a = f32(rng.uniform(-0.99, 0.99, (2, 64, 64)))
    x = f32(rng.standard_normal((2, 64, 64)) * 0.5)
    dy = f32(rng.standard_normal((2, 64, 64)))
    y, fs = orc.rglru_forward(a, x)
    da, dx, _ = orc.rglru_backward(dy, a, x)
    return dict(a=a, x=x, dy=dy, y=y, final=fs, da=da, dx=dx)


def rotlru_small():
    """test_v2_rotlru.py:43-60 shape (1, 96, 16): D = 32 edge, three segments."""
    rng = np.random.default_rng(104)
    th = rng.uniform(0.0, np.pi, (1, 96, 16))
    a = f32(rng.uniform(0.0, 0.99, (1, 96, 16)))
    cs, sn = f32(np.cos(th)), f32(np.sin(th))
    x = f32(rng.standard_normal((1, 96, 32)) * 0.5)
    dy = f32(rng.standard_normal((1, 96, 32)))
    y, fs = orc.rotlru_forward(a, cs, sn, x)
    da, dcs, dsn, dx, _ = orc.rotlru_backward(dy, a, cs, sn, x)
    return dict(a=a, cs=cs, sn=sn, x=x, dy=dy, y=y, final=fs, da=da, dcs=dcs, dsn=dsn, dx=dx)


FIXTURES = {
    "ssd_c0": ssd_c0,
    "ssd_ref_shape": ssd_ref_shape,
    "gla_small": gla_small,
    "rglru_small": rglru_small,
    "rotlru_small": rotlru_small,
}


def main():
    for name, fn in FIXTURES.items():
        arrays = fn()
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
