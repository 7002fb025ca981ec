"""Bit-exact repeatability of the scans (MI355X only).

Every pass is deterministic by construction: fixed reduction orders, no
floating-point atomics, and hand-offs between workgroups that each wait for
exactly one producer.  A race between waves of a workgroup (a missing LDS
barrier) or between workgroups would show up as run-to-run differences far
below the parity bars, so these tests demand bit equality:
  * two eager runs of a forward + backward through the C ABI (bench.py's
    workloads: the BASELINE configurations and the other kernel modes);
  * a HIP graph of the same calls, replayed three times with eager work in
    between (the outputs and workspaces are overwritten with 0xFF bytes before
    each replay), against the eager result.
"""
from __future__ import annotations

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu

CASES = [
    # (bench workload maker, config); the chunked SSD/GLA modes: direct (c1, c2),
    # whole head (B96 forward), pipelined (B96 backward, c4-like N = 128 with the
    # per-head adjoint scan); the tiled RG-LRU / rotLRU passes (config 3)
    ("ssd", dict(B=3, L=512, H=12, Dh=64, N=16, seg=32)),
    ("gla", dict(B=3, L=512, H=12, Dh=64, seg=32)),
    ("ssd", dict(B=96, L=512, H=12, Dh=64, N=16, seg=32)),
    ("gla", dict(B=96, L=512, H=12, Dh=64, seg=32)),
    ("ssd", dict(B=8, L=1024, H=80, Dh=64, N=128, seg=32)),
    ("rglru", dict(B=8, L=4096, D=2560, seg=32)),
    ("rglru_gated", dict(B=8, L=4096, D=2560, seg=32)),
    ("rotlru", dict(B=8, L=4096, D=2560, seg=32)),
    ("rotlru_theta", dict(B=8, L=4096, D=2560, seg=32)),
    # the per-chunk fp32-MFMA kernels: a rate per (head, n), fp32 SSD, fp32 GLA
    ("ssd", dict(B=3, L=512, H=12, Dh=64, N=16, seg=32, dense=True)),
    ("ssd", dict(B=3, L=512, H=12, Dh=64, N=16, seg=32, dtype="f32")),
    ("gla", dict(B=3, L=512, H=12, Dh=64, seg=32, dtype="f32")),
    # the same at the reference's published shape (wide states: d streamed in blocks)
    ("ssd", dict(B=3, L=512, H=12, Dh=128, N=64, seg=32, dense=True)),
    ("gla", dict(B=3, L=512, H=12, Dh=128, seg=32, dtype="f32")),
    # the published shape in bf16 with a per-head rate: the wide direct mode
    # (block-owned sums over the other chunks, the adjoint through the workspace)
    ("ssd", dict(B=3, L=512, H=12, Dh=128, N=64, seg=32)),
    ("gla", dict(B=3, L=512, H=12, Dh=128, seg=32)),
]
MAKERS = {"ssd": bench.make_ssd, "gla": bench.make_gla, "rglru": bench.make_rglru,
          "rglru_gated": bench.make_rglru_gated, "rotlru": bench.make_rotlru,
          "rotlru_theta": bench.make_rotlru_theta}


def _results(w):
    return {k: v.clone() for k, v in w["out"].items() if v is not None and not k.startswith("ws")}


def _scribble(w):
    for v in w["out"].values():
        if v is not None:
            v.view(torch.uint8).fill_(0xFF)


def _diff(a, b):
    bad = [k for k in a if not torch.equal(a[k].view(torch.uint8), b[k].view(torch.uint8))]
    return bad


@pytest.mark.parametrize("name,cfg", CASES, ids=[f"{n}-" + "-".join(f"{k}{v}" for k, v in c.items()) for n, c in CASES])
def test_bit_exact_repeat_and_graph_replay(name, cfg):
    print(f"[case] determinism {name} {cfg}", flush=True)
    dev = torch.device("cuda:0")
    w = MAKERS[name](cfg, dev, torch.bfloat16)
    stream = torch.cuda.Stream(dev)
    with torch.cuda.stream(stream):
        w["fwd"]()
        w["bwd"]()
    torch.cuda.synchronize()
    first = _results(w)
    _scribble(w)                              # on the default stream: finish it before the next run
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        w["fwd"]()
        w["bwd"]()
    torch.cuda.synchronize()
    second = _results(w)
    assert not _diff(first, second), f"eager runs differ in {_diff(first, second)}"

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        w["fwd"]()
        w["bwd"]()
    for rep in range(3):
        _scribble(w)                          # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = _results(w)
        bad = _diff(first, got)
        assert not bad, f"graph replay {rep} differs from the eager run in {bad}"
    del graph
