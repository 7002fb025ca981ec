"""Hand-off order of the RG-LRU / rotLRU tiled chained scans — CPU only.

The tile kernels (rglru.hip, rotlru.hip) wait for the state (forward) or the
adjoint (backward) of the tile of the same channels one step tile earlier
(later).  The wait always ends only if that predecessor's workgroup took a
smaller ticket (it is then resident or finished).  These tests read the
library's own ticket -> tile map (rr_tile_schedule, the same functions the
kernels call) for the BASELINE config-3 grids and ragged shapes, and check:
  * the map is a bijection onto the B*G x K tiles;
  * every predecessor holds a smaller ticket;
  * the backward reads checkpoint rows below B*nC only (waves past L read
    nothing), for every checkpoint interval T in {1, 2, 4, ..., 32}.
"""
import numpy as np
import pytest

from mlx_recurrence_amd import _lib

F32, BF16, F16 = 0, 1, 2
RGLRU, RGLRU_GATED, ROTLRU = 0, 1, 2

SHAPES = [
    # (scan, B, L, D, seg, dtype)
    (RGLRU, 8, 4096, 2560, 32, BF16),
    (RGLRU_GATED, 8, 4096, 2560, 32, BF16),
    (ROTLRU, 8, 4096, 1280, 32, BF16),     # 1280 pairs
    (RGLRU, 3, 200, 64, 8, F32),           # ragged L (not a tile multiple), T = 8
    (RGLRU, 2, 96, 96, 16, F16),           # ragged D
    (RGLRU_GATED, 3, 200, 96, 8, F32),
    (ROTLRU, 2, 160, 48, 16, F32),         # Dp not a tile multiple, T = 16
    (ROTLRU, 1, 96, 16, 32, BF16),
    (RGLRU, 1, 30, 32, 3, F32),            # T = 1
    (RGLRU, 2, 1000, 320, 40, BF16),       # seg 40 -> T = 8
]


def _check_schedule(scan, pass_, B, L, D, seg, dtype):
    k, g, worst = _lib.tile_schedule(scan, pass_, B, L, D, seg, dtype)
    n = k.size
    K = int(k.max()) + 1
    nGrp = int(g.max()) + 1
    assert n == K * nGrp
    ticket = np.full((nGrp, K), -1, dtype=np.int64)
    ticket[g, k] = np.arange(n)
    assert (ticket >= 0).all(), "some tile has no ticket"
    assert len(set(zip(g.tolist(), k.tolist()))) == n, "two tickets run one tile"
    if pass_ == 0:   # waits for tile k - 1 of the same channels
        assert (ticket[:, 1:] > ticket[:, :-1]).all()
    else:            # waits for tile k + 1
        assert (ticket[:, :-1] > ticket[:, 1:]).all()
    return worst


@pytest.mark.parametrize("scan,B,L,D,seg,dtype", SHAPES)
@pytest.mark.parametrize("pass_", [0, 1])
def test_predecessor_holds_smaller_ticket(scan, B, L, D, seg, dtype, pass_):
    _check_schedule(scan, pass_, B, L, D, seg, dtype)


@pytest.mark.parametrize("scan", [RGLRU, RGLRU_GATED, ROTLRU])
@pytest.mark.parametrize("seg", [1, 2, 4, 8, 16, 32, 96])
@pytest.mark.parametrize("nC", [1, 3, 5, 7])
def test_backward_checkpoint_rows_in_bounds(scan, seg, nC):
    """Ragged L = nC * seg: the last step tile has padding waves past L."""
    B, L, D = 2, nC * seg, 96
    worst = _check_schedule(scan, 1, B, L, D, seg, F32)
    T = _lib.chunk_len(L, seg)
    assert worst < B * (L // T)


def test_schedule_rejects_bad_arguments():
    with pytest.raises(ValueError):
        _lib.tile_schedule(3, 0, 1, 64, 64, 32, F32)
    with pytest.raises(ValueError):
        _lib.tile_schedule(0, 0, 1, 30, 64, 32, F32)
