"""Workspace bounds of the chunked SSD passes — CPU only.

The adjoint scan writes one adjoint per run of R chunks of each head into the
backward workspace, the pipelined and pair chunk kernels read them back, and
every backward workgroup writes a dA partial there.  A slot computed past the
end of the workspace is an out-of-bounds write on the GPU (the pair mode's
first run did exactly that: its scan spaced each head's slots nC apart where
the workspace holds ceil(nC / R)).  These tests ask the library for the
largest workspace byte its kernels touch (rr_ssd_workspace_extent: the grids
walked with the kernels' own workgroup decode and slot arithmetic) and check
it against the size the library asks callers for (rr_ssd_workspace_bytes),
for BASELINE config 4, ragged even chunk counts in pair mode, and the other
modes' shapes.
"""
import pytest

from mlx_recurrence_amd import _lib

BF16 = 1
ALIGN = 256   # every workspace part starts 256-byte aligned

SHAPES = [
    # (B, L, H, Dh, N) at seg 32, bf16, a per-head A (the chunked kernels)
    (8, 4096, 80, 64, 128),    # pair mode (nC 128)
    (4, 64, 80, 64, 128),      # pair mode, nC 2
    (4, 192, 80, 64, 64),      # pair mode, nC 6
    (1, 320, 320, 32, 128),    # pair mode, nC 10, Dh 32
    (5, 1088, 64, 64, 64),     # pair mode, nC 34
    (4, 160, 80, 64, 128),     # nC 5 (odd): per-chunk adjoints from the scan
    (2, 1056, 4, 64, 64),      # nC 33, few heads: aggregate + adjoint-pass kernels
    (3, 512, 12, 64, 16),      # sum mode
    (3, 512, 12, 64, 64),      # per-chunk mode, wide state, few heads
    (2, 128, 3, 128, 64),      # wide direct mode (nC 4), Dh 128
    (3, 512, 12, 128, 64),     # wide direct mode: the reference's published shape
    (2, 256, 6, 64, 128),      # Dh 64 N 128, short heads: pipelined
    (4, 512, 16, 128, 64),     # Dh 128, 1024 chunk workgroups: per-chunk mode
    (96, 512, 12, 64, 16),     # SSD c1 shape at B 96: per-chunk with the scan
]


@pytest.mark.parametrize("B,L,H,Dh,N", SHAPES)
@pytest.mark.parametrize("pass_", [0, 1])
def test_kernels_stay_inside_the_workspace(B, L, H, Dh, N, pass_):
    lib = _lib.load()
    need = int(lib.rr_ssd_workspace_bytes(B, L, H, Dh, N, 32, 0, BF16, pass_))
    ext = _lib.ssd_workspace_extent(B, L, H, Dh, N, 32, 0, BF16, pass_)
    assert ext >= 0
    assert ext <= need, f"kernels touch {ext} bytes of a {need}-byte workspace"
    if pass_ == 1:
        # every part of the backward workspace is used up to its alignment padding
        assert need - ext < ALIGN, (need, ext)


def test_pair_mode_bound_detects_the_old_slot_spacing():
    """The bound is tight enough to catch the pair mode's old slot spacing:
    at config 4 the last head's last adjoint, with slots nC (not nC / 2)
    apart per head, lies past the end of the workspace."""
    B, L, H, Dh, N = 8, 4096, 80, 64, 128
    nC, R = L // 32, 2
    lib = _lib.load()
    need = int(lib.rr_ssd_workspace_bytes(B, L, H, Dh, N, 32, 0, BF16, 1))
    ext = _lib.ssd_workspace_extent(B, L, H, Dh, N, 32, 0, BF16, 1)
    state = Dh * N * 4
    agg_end_now = ext                       # the adjoints are the workspace's last part
    last_slot_now = (B * H - 1) * (nC // R) + nC // R - 1
    last_slot_old = (B * H - 1) * nC + nC // R - 1
    agg_begin = agg_end_now - (last_slot_now + 1) * state
    assert agg_begin >= 0
    assert agg_begin + (last_slot_old + 1) * state > need


def test_extent_for_valu_engine_calls_and_bad_arguments():
    # a dense A_neg [H, N] or fp32 inputs run other kernels: no bound from this walk
    assert _lib.ssd_workspace_extent(3, 512, 12, 64, 16, 32, 1, BF16, 1) == -1
    assert _lib.ssd_workspace_extent(3, 512, 12, 64, 16, 32, 0, 0, 1) == -1   # fp32 inputs
    assert _lib.ssd_workspace_extent(0, 512, 12, 64, 16, 32, 0, BF16, 1) == -1
    assert _lib.ssd_workspace_extent(3, 512, 12, 64, 16, 32, 0, BF16, 2) == -1


def test_wide_direct_mode_workspace_at_the_published_shape():
    """The reference's published shape (B3 L512 H12 Dh128 N64, bf16, a rate per
    head) runs the wide direct mode: one kernel per pass, so the forward needs
    no workspace, and the backward holds the dA partials [B,H,nC,N] and one
    adjoint [Dh,N] per chunk (du's operand rows), each part 256-byte aligned.
    Past 768 chunk workgroups the same state takes the resident forward (no
    workspace) and the pipelined backward (per-chunk decays as well)."""
    lib = _lib.load()
    B, L, H, Dh, N = 3, 512, 12, 128, 64
    nC = L // 32

    def al(nbytes):
        return (nbytes + ALIGN - 1) // ALIGN * ALIGN

    assert int(lib.rr_ssd_workspace_bytes(B, L, H, Dh, N, 32, 0, BF16, 0)) == 0
    assert int(lib.rr_ssd_workspace_bytes(B, L, H, Dh, N, 32, 0, BF16, 1)) == \
        al(B * H * nC * N * 4) + al(B * H * nC * Dh * N * 4)
    assert int(lib.rr_gla_workspace_bytes(B, L, H, Dh, 32, BF16, 0)) == 0
    assert int(lib.rr_gla_workspace_bytes(B, L, H, Dh, 32, BF16, 1)) == al(B * H * nC * Dh * Dh * 4)
    # 5 x 12 x 16 = 960 chunk workgroups
    assert int(lib.rr_ssd_workspace_bytes(5, L, H, Dh, N, 32, 0, BF16, 0)) == 0
    assert int(lib.rr_ssd_workspace_bytes(5, L, H, Dh, N, 32, 0, BF16, 1)) == \
        al(5 * H * nC * 4) + al(5 * H * nC * N * 4) + al(5 * H * nC * Dh * N * 4)
