"""The C ABI library loads, exports every symbol include/recurrence.h declares,
and rejects invalid calls before touching the GPU — CPU only (no kernel runs)."""
import ctypes
import pathlib
import re

import pytest

from mlx_recurrence_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "recurrence.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(rr_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (run mlx-recurrence_amd/build.py)")
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    declared = _declared()
    assert declared, "no rr_* declarations parsed from the header"
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared but not exported: {missing}"
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared, "ctypes signature table out of sync with the header"


def test_abi_version(lib):
    assert lib.rr_abi_version() == 12


@pytest.mark.parametrize("L,seg,T", [(512, 32, 32), (96, 16, 16), (128, 64, 32), (96, 48, 16),
                                     (30, 3, 1), (30, 32, 0), (32, 0, 0), (4096, 32, 32), (64, 8, 8)])
def test_chunk_len(lib, L, seg, T):
    assert lib.rr_chunk_len(L, seg) == T


def _call_rglru_fwd(L, D, seg, dtype=0, null=False):
    p = None if null else ctypes.c_void_p(16)  # never dereferenced: validation fails first
    return _lib.load().rr_rglru_fwd(p, p, dtype, 1, L, D, seg, None, p, p, p, 1 << 30, None)


def test_rejects_bad_shapes_before_launch(lib):
    assert _call_rglru_fwd(30, 32, 32) == _lib.RR_EINVAL
    assert b"must be divisible by seg=32" in lib.rr_last_error()
    assert _call_rglru_fwd(32, 16, 32) == _lib.RR_EINVAL
    assert b"D=16 must be a multiple of 32" in lib.rr_last_error()
    assert _call_rglru_fwd(32, 32, 0) == _lib.RR_EINVAL
    assert b"seg must be positive" in lib.rr_last_error()
    assert _call_rglru_fwd(32, 32, 32, dtype=7) == _lib.RR_EINVAL
    assert _call_rglru_fwd(32, 32, 32, null=True) == _lib.RR_EINVAL
    assert b"null pointer" in lib.rr_last_error()


def test_ssd_gla_validation(lib):
    p = ctypes.c_void_p(16)
    rc = lib.rr_ssd_fwd(p, p, p, p, p, 1, 0, 1, 30, 2, 32, 8, 32, None, p, p, None, 0, None)
    assert rc == _lib.RR_EINVAL and b"L=30" in lib.rr_last_error()
    rc = lib.rr_gla_fwd(p, p, p, p, 0, 1, 32, 2, 16, 32, None, p, p, None, 0, None)
    assert rc == _lib.RR_EINVAL and b"Dh=16" in lib.rr_last_error()
    rc = lib.rr_ssd_fwd(p, p, p, p, p, 3, 0, 1, 32, 2, 32, 8, 32, None, p, p, None, 0, None)
    assert rc == _lib.RR_EINVAL and b"A_stride_n" in lib.rr_last_error()
    # too-small workspace is reported, not overrun
    need = lib.rr_ssd_workspace_bytes(2, 64, 2, 64, 8, 32, 1, 0, 1)
    if need:
        rc = lib.rr_ssd_bwd(p, None, p, p, p, p, p, 1, 0, 2, 64, 2, 64, 8, 32, None, p, p, p, p, p, p, 1, None,
                            p, need - 1, None)
        assert rc == _lib.RR_EWORKSPACE
        rc = lib.rr_ssd_bwd(p, None, p, p, p, p, p, 1, 0, 2, 64, 2, 64, 8, 32, None, p, p, p, p, p, p, 2, None,
                            p, need, None)
        assert rc == _lib.RR_EINVAL and b"dA_stride_n" in lib.rr_last_error()
    need = lib.rr_rglru_workspace_bytes(2, 256, 64, 32, 1, 0)
    assert need > 0
    rc = lib.rr_rglru_fwd(p, p, 1, 2, 256, 64, 32, None, p, p, p, need - 1, None)
    assert rc == _lib.RR_EWORKSPACE


def test_ssd_bwd_noalloc_rejects_beyond_its_scratch(lib):
    """The no-allocation SSD backward refuses calls whose workspace exceeds its
    16 MiB static scratch, before touching the device (B = 96: 75 MB)."""
    p = ctypes.c_void_p(16)  # never dereferenced: the size check fails first
    need = lib.rr_ssd_workspace_bytes(96, 512, 12, 64, 16, 32, 0, 1, 1)
    assert need > (16 << 20)
    rc = lib.rr_ssd_bwd_noalloc(p, None, p, p, p, p, p, 0, 1, 96, 512, 12, 64, 16, 32, None, p, p, p, p, p, p,
                                1, None, None)
    assert rc == _lib.RR_EUNSUPPORTED and b"16777216-byte device scratch" in lib.rr_last_error()
    assert lib.rr_ssd_workspace_bytes(3, 512, 12, 64, 16, 32, 0, 1, 1) <= (16 << 20)   # config 1 fits
    rc = lib.rr_ssd_bwd_noalloc(p, None, p, p, p, p, p, 0, 1, 3, 30, 12, 64, 16, 32, None, p, p, p, p, p, p,
                                1, None, None)
    assert rc == _lib.RR_EINVAL and b"L=30" in lib.rr_last_error()


def test_gdn_validation(lib):
    """Gated DeltaNet entry points: shape rules and the kernels' Dh / interval
    limits are reported before any launch."""
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.rr_gdn_fwd(p, p, p, p, p, 0, 1, 30, 2, 64, 32, None, p, p, None, 0, None)
    assert rc == _lib.RR_EINVAL and b"L=30" in lib.rr_last_error()
    rc = lib.rr_gdn_fwd(p, p, p, p, p, 0, 1, 64, 2, 128, 32, None, p, p, None, 0, None)
    assert rc == _lib.RR_EUNSUPPORTED and b"Dh must be 32 or 64" in lib.rr_last_error()
    rc = lib.rr_gdn_fwd(p, p, p, p, p, 0, 1, 12, 2, 64, 4, None, p, p, None, 0, None)
    assert rc == _lib.RR_EUNSUPPORTED and b"multiple of 8" in lib.rr_last_error()
    rc = lib.rr_gdn_fwd(p, p, p, p, None, 0, 1, 64, 2, 64, 32, None, p, p, None, 0, None)
    assert rc == _lib.RR_EINVAL and b"null pointer" in lib.rr_last_error()
    rc = lib.rr_gdn_bwd(p, None, p, p, p, p, p, 0, 1, 64, 2, 64, 32, None, p, p, p, None, p, p, None, p, 1 << 30,
                        None)
    assert rc == _lib.RR_EINVAL and b"null pointer" in lib.rr_last_error()
    need = lib.rr_gdn_workspace_bytes(1, 64, 2, 64, 32, 0)
    assert need == 1 * 2 * 2 * 64 * 64 * 4
    rc = lib.rr_gdn_bwd(p, None, p, p, p, p, p, 0, 1, 64, 2, 64, 32, None, p, p, p, p, p, p, None, p, need - 1, None)
    assert rc == _lib.RR_EWORKSPACE
    q_odd = ctypes.c_void_p(24)
    rc = lib.rr_gdn_fwd(q_odd, p, p, p, p, 0, 1, 64, 2, 64, 32, None, p, p, None, 0, None)
    assert rc == _lib.RR_EINVAL and b"16-byte aligned" in lib.rr_last_error()
    # the chunkwise forward's workspace: bf16, Dh 64, T 32 only (one pack per chunk)
    fneed = lib.rr_gdn_fwd_workspace_bytes(2, 64, 3, 64, 32, 1)
    assert fneed > 0 and fneed % (2 * 3 * 2) == 0
    assert lib.rr_gdn_fwd_workspace_bytes(2, 64, 3, 64, 32, 0) == 0     # fp32: sequential
    assert lib.rr_gdn_fwd_workspace_bytes(2, 64, 3, 32, 32, 1) == 0     # Dh 32
    assert lib.rr_gdn_fwd_workspace_bytes(2, 64, 3, 64, 16, 1) == 0     # T 16
    assert lib.rr_gdn_fwd_workspace_bytes(2, 30, 3, 64, 32, 1) == 0     # invalid L
    rc = lib.rr_gdn_fwd(p, p, p, p, p, 1, 2, 64, 3, 64, 32, None, p, p, p, fneed - 1, None)
    assert rc == _lib.RR_EWORKSPACE
    rc = lib.rr_gdn_fwd(p, p, p, p, p, 1, 2, 64, 3, 64, 32, None, p, p, ctypes.c_void_p(24), fneed, None)
    assert rc == _lib.RR_EWORKSPACE and b"misaligned" in lib.rr_last_error()
    rc = lib.rr_gdn_fwd(p, p, p, p, p, 0, 2, 64, 3, 64, 32, None, p, p, p, 1 << 30, None)
    assert rc == _lib.RR_EINVAL and b"chunkwise form" in lib.rr_last_error()
