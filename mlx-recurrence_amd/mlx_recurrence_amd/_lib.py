"""ctypes binding of librecurrence_gfx950.so (C ABI declared in include/recurrence.h).

The library is built ahead of time for gfx950 by ``mlx-recurrence_amd/build.py``
and loaded from this directory.  There is no fallback: if the library is
missing or the tensors are not on a ROCm device the call raises.

Every wrapper here takes torch tensors, checks device/dtype/contiguity, and
passes raw device pointers plus the current stream of the tensors' device.
"""
from __future__ import annotations

import ctypes
import functools
import os
import pathlib

import torch

LIB_NAME = "librecurrence_gfx950.so"
# MLX_RECURRENCE_AMD_LIB names another build of the library to load instead
# (the host-sanitizer build that the CPU tests of the C ABI run against).
LIB_PATH = pathlib.Path(os.environ.get("MLX_RECURRENCE_AMD_LIB") or
                        pathlib.Path(__file__).resolve().parent / LIB_NAME)

RR_OK = 0
RR_EINVAL = 1
RR_EUNSUPPORTED = 2
RR_EHIP = 3
RR_EWORKSPACE = 4

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGS = {
    "rr_abi_version": (_c_int, []),
    "rr_last_error": (ctypes.c_char_p, []),
    "rr_chunk_len": (_c_i64, [_c_i64, _c_i64]),
    "rr_async_status": (_c_int, []),
    "rr_tile_schedule": (_c_i64, [_c_int, _c_int] + [_c_i64] * 4 + [_c_int] + [_c_ptr] * 3 + [_c_i64]),
    "rr_ssd_workspace_bytes": (_c_size, [_c_i64] * 7 + [_c_int, _c_int]),
    "rr_ssd_workspace_extent": (_c_i64, [_c_i64] * 7 + [_c_int, _c_int]),
    "rr_ssd_fwd": (_c_int, [_c_ptr] * 5 + [_c_i64, _c_int] + [_c_i64] * 6 + [_c_ptr] * 4 + [_c_size, _c_ptr]),
    "rr_ssd_bwd": (_c_int, [_c_ptr] * 7 + [_c_i64, _c_int] + [_c_i64] * 6 + [_c_ptr] * 7 + [_c_i64]
                   + [_c_ptr] * 2 + [_c_size, _c_ptr]),
    "rr_ssd_bwd_noalloc": (_c_int, [_c_ptr] * 7 + [_c_i64, _c_int] + [_c_i64] * 6 + [_c_ptr] * 7 + [_c_i64]
                           + [_c_ptr] * 2),
    "rr_gla_workspace_bytes": (_c_size, [_c_i64] * 5 + [_c_int, _c_int]),
    "rr_gla_fwd": (_c_int, [_c_ptr] * 4 + [_c_int] + [_c_i64] * 5 + [_c_ptr] * 4 + [_c_size, _c_ptr]),
    "rr_gla_bwd": (_c_int, [_c_ptr] * 6 + [_c_int] + [_c_i64] * 5 + [_c_ptr] * 8 + [_c_size, _c_ptr]),
    "rr_rglru_workspace_bytes": (_c_size, [_c_i64] * 4 + [_c_int, _c_int]),
    "rr_rglru_fwd": (_c_int, [_c_ptr] * 2 + [_c_int] + [_c_i64] * 4 + [_c_ptr] * 4 + [_c_size, _c_ptr]),
    "rr_rglru_bwd": (_c_int, [_c_ptr] * 4 + [_c_int] + [_c_i64] * 4 + [_c_ptr] * 6 + [_c_size, _c_ptr]),
    "rr_rglru_gated_workspace_bytes": (_c_size, [_c_i64] * 4 + [_c_int, _c_int]),
    "rr_rglru_gated_fwd": (_c_int, [_c_ptr] * 4 + [ctypes.c_float, _c_int] + [_c_i64] * 4 + [_c_ptr] * 4
                           + [_c_size, _c_ptr]),
    "rr_rglru_gated_bwd": (_c_int, [_c_ptr] * 6 + [ctypes.c_float, _c_int] + [_c_i64] * 4 + [_c_ptr] * 8
                           + [_c_size, _c_ptr]),
    "rr_rotlru_workspace_bytes": (_c_size, [_c_i64] * 4 + [_c_int, _c_int]),
    "rr_rotlru_fwd": (_c_int, [_c_ptr] * 4 + [_c_int] + [_c_i64] * 4 + [_c_ptr] * 4 + [_c_size, _c_ptr]),
    "rr_rotlru_bwd": (_c_int, [_c_ptr] * 6 + [_c_int] + [_c_i64] * 4 + [_c_ptr] * 8 + [_c_size, _c_ptr]),
    "rr_rotlru_theta_fwd": (_c_int, [_c_ptr] * 3 + [_c_int] + [_c_i64] * 4 + [_c_ptr] * 4 + [_c_size, _c_ptr]),
    "rr_rotlru_theta_bwd": (_c_int, [_c_ptr] * 5 + [_c_int] + [_c_i64] * 4 + [_c_ptr] * 7 + [_c_size, _c_ptr]),
    "rr_ssd_step": (_c_int, [_c_ptr] * 5 + [_c_i64, _c_int] + [_c_i64] * 4 + [_c_ptr] * 3),
    "rr_gla_step": (_c_int, [_c_ptr] * 4 + [_c_int] + [_c_i64] * 3 + [_c_ptr] * 3),
    "rr_rglru_step": (_c_int, [_c_ptr] * 2 + [_c_int] + [_c_i64] * 2 + [_c_ptr] * 3),
    "rr_rotlru_step": (_c_int, [_c_ptr] * 4 + [_c_int] + [_c_i64] * 2 + [_c_ptr] * 3),
    "rr_gdn_fwd": (_c_int, [_c_ptr] * 5 + [_c_int] + [_c_i64] * 5 + [_c_ptr] * 4 + [_c_size, _c_ptr]),
    "rr_gdn_fwd_workspace_bytes": (_c_size, [_c_i64] * 5 + [_c_int]),
    "rr_gdn_workspace_bytes": (_c_size, [_c_i64] * 5 + [_c_int]),
    "rr_gdn_bwd": (_c_int, [_c_ptr] * 7 + [_c_int] + [_c_i64] * 5 + [_c_ptr] * 9 + [_c_size, _c_ptr]),
}

EXPORTED_SYMBOLS = tuple(_SIGS)

_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_NAME} not found at {LIB_PATH}; build it with "
            "`python mlx-recurrence_amd/build.py` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def abi_version() -> int:
    return load().rr_abi_version()


_AUTOGRAD_UNSET = object()
_autograd_mod = _AUTOGRAD_UNSET


def autograd_ext():
    """The C++ autograd bindings (module mlx_recurrence_amd._autograd, built by
    build.py next to the library), or None where they are not built.  Both
    bindings call the same kernels through the same C ABI."""
    global _autograd_mod
    if _autograd_mod is _AUTOGRAD_UNSET:
        load()   # the library first: the extension links this same file
        try:
            from . import _autograd as mod
        except ImportError:
            mod = None
        if mod is not None and mod.abi_version() != load().rr_abi_version():
            mod = None   # built against another revision of the library
        _autograd_mod = mod
    return _autograd_mod


def chunk_len(L: int, seg: int) -> int:
    return chunk_len_cached(int(L), int(seg))


def async_status() -> None:
    """Synchronise the current device and raise RuntimeError if a kernel since
    the last check reported an error after its launch returned (an expired
    tile hand-off wait: that pass's results are NaN)."""
    _check(load().rr_async_status(), "rr_async_status")


def tile_schedule(scan: int, pass_: int, B: int, L: int, D: int, seg: int, dtype: int):
    """(tile_k, tile_grp, max_ckpt_row) per workgroup ticket of an RG-LRU
    (scan 0), gated RG-LRU (1) or rotLRU (2, D = pairs) pass, as numpy arrays."""
    import numpy as np
    lib = load()
    n = int(lib.rr_tile_schedule(scan, pass_, B, L, D, seg, dtype, None, None, None, 0))
    if n < 0:
        raise ValueError(lib.rr_last_error().decode())
    k = np.empty(n, dtype=np.int32)
    g = np.empty(n, dtype=np.int32)
    worst = ctypes.c_int64(0)
    lib.rr_tile_schedule(scan, pass_, B, L, D, seg, dtype, k.ctypes.data_as(_c_ptr), g.ctypes.data_as(_c_ptr),
                         ctypes.byref(worst), n)
    return k, g, int(worst.value)


def ssd_workspace_extent(B: int, L: int, H: int, Dh: int, N: int, seg: int, a_stride_n: int, dtype: int,
                         pass_: int) -> int:
    """One past the largest workspace byte the chunked (bf16) SSD kernels of a
    pass touch (walked over their grids by the library), or -1 where the call
    runs on the fp32-MFMA or VALU paths (fixed workspace regions)."""
    return int(load().rr_ssd_workspace_extent(B, L, H, Dh, N, seg, a_stride_n, dtype, pass_))


def _check(rc: int, what: str) -> None:
    if rc == RR_OK:
        return
    msg = load().rr_last_error().decode(errors="replace")
    if rc in (RR_EINVAL, RR_EWORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def ptr(t: torch.Tensor | None):
    """Device address of a tensor (an int; ctypes passes it as void*), or None."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor):
    """The current stream of t's device as a raw hipStream_t address."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index if t.device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(t.device).cuda_stream


class _NoGuard:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_GUARD = _NoGuard()


def device_guard(dev: torch.device):
    """torch.cuda.device(dev) when dev is not the current device (the library
    looks up per-device addresses on the current device), else a no-op."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(dev)


def require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "mlx_recurrence_amd kernels run on a ROCm GPU; got a tensor on "
                f"{t.device} (use the *_scan_reference functions for CPU tensors)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"all tensors must be on one device, got {dev} and {t.device}")
    return dev


def prep(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Contiguous, 16-byte aligned, of the requested dtype."""
    if t.dtype != dtype:
        t = t.to(dtype)
    if not t.is_contiguous():
        t = t.contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t


def common_dtype(*tensors: torch.Tensor) -> torch.dtype:
    dt = tensors[0].dtype
    for t in tensors[1:]:
        dt = torch.promote_types(dt, t.dtype)
    if dt not in DTYPE_CODE:
        if dt.is_floating_point:
            dt = torch.float32
        else:
            raise TypeError(f"unsupported input dtype {dt}; use float32, bfloat16 or float16")
    return dt


@functools.lru_cache(maxsize=1024)
def _ws_bytes(fn_name: str, args: tuple) -> int:
    return int(getattr(load(), fn_name)(*args))


@functools.lru_cache(maxsize=1024)
def chunk_len_cached(L: int, seg: int) -> int:
    return int(load().rr_chunk_len(L, seg))


def _alloc_ws(n: int, device) -> torch.Tensor | None:
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


# ---------------------------------------------------------------- SSD
def ssd_workspace(B, L, H, Dh, N, seg, a_stride_n, dtype, pass_, device) -> torch.Tensor | None:
    n = _ws_bytes("rr_ssd_workspace_bytes", (B, L, H, Dh, N, seg, a_stride_n, DTYPE_CODE[dtype], pass_))
    return _alloc_ws(n, device)


def ssd_fwd(u, delta, Bm, Cm, A, a_stride_n, h0, seg, y, ckpt, ws):
    """A is [H, N] fp32 (a_stride_n=1) or one rate per head [H] (a_stride_n=0)."""
    B, L, H, Dh = u.shape
    N = Bm.shape[-1]
    rc = load().rr_ssd_fwd(
        ptr(u), ptr(delta), ptr(Bm), ptr(Cm), ptr(A), a_stride_n, DTYPE_CODE[u.dtype],
        B, L, H, Dh, N, seg, ptr(h0), ptr(y), ptr(ckpt), ptr(ws),
        0 if ws is None else ws.numel(), stream_of(u))
    _check(rc, "rr_ssd_fwd")


def ssd_bwd(dy, dfinal, u, delta, Bm, Cm, A, a_stride_n, h0, ckpt, seg, du, ddelta, dB, dC, dA, dh0, ws):
    """rr_ssd_bwd; dA is [H, N] (dense gradient) or [H] (per-head gradient,
    summed over n by the library)."""
    B, L, H, Dh = u.shape
    N = Bm.shape[-1]
    rc = load().rr_ssd_bwd(
        ptr(dy), ptr(dfinal), ptr(u), ptr(delta), ptr(Bm), ptr(Cm), ptr(A), a_stride_n,
        DTYPE_CODE[u.dtype], B, L, H, Dh, N, seg, ptr(h0), ptr(ckpt), ptr(du),
        ptr(ddelta), ptr(dB), ptr(dC), ptr(dA), 0 if dA.ndim == 1 else 1, ptr(dh0), ptr(ws),
        0 if ws is None else ws.numel(), stream_of(u))
    _check(rc, "rr_ssd_bwd")


def ssd_bwd_noalloc(dy, dfinal, u, delta, Bm, Cm, A, a_stride_n, h0, ckpt, seg, du, ddelta, dB, dC, dA, dh0):
    """rr_ssd_bwd_noalloc: the backward with the library's static device scratch
    as workspace (no allocation; calls overlapping on one device race)."""
    B, L, H, Dh = u.shape
    N = Bm.shape[-1]
    rc = load().rr_ssd_bwd_noalloc(
        ptr(dy), ptr(dfinal), ptr(u), ptr(delta), ptr(Bm), ptr(Cm), ptr(A), a_stride_n,
        DTYPE_CODE[u.dtype], B, L, H, Dh, N, seg, ptr(h0), ptr(ckpt), ptr(du),
        ptr(ddelta), ptr(dB), ptr(dC), ptr(dA), 0 if dA.ndim == 1 else 1, ptr(dh0), stream_of(u))
    _check(rc, "rr_ssd_bwd_noalloc")


# ---------------------------------------------------------------- GLA
def gla_workspace(B, L, H, Dh, seg, dtype, pass_, device) -> torch.Tensor | None:
    n = _ws_bytes("rr_gla_workspace_bytes", (B, L, H, Dh, seg, DTYPE_CODE[dtype], pass_))
    return _alloc_ws(n, device)


def gla_fwd(q, k, v, g, h0, seg, y, ckpt, ws):
    B, L, H, Dh = q.shape
    rc = load().rr_gla_fwd(
        ptr(q), ptr(k), ptr(v), ptr(g), DTYPE_CODE[q.dtype], B, L, H, Dh, seg,
        ptr(h0), ptr(y), ptr(ckpt), ptr(ws), 0 if ws is None else ws.numel(), stream_of(q))
    _check(rc, "rr_gla_fwd")


def gla_bwd(dy, dfinal, q, k, v, g, h0, ckpt, seg, dq, dk, dv, dg, dh0, ws):
    B, L, H, Dh = q.shape
    rc = load().rr_gla_bwd(
        ptr(dy), ptr(dfinal), ptr(q), ptr(k), ptr(v), ptr(g), DTYPE_CODE[q.dtype],
        B, L, H, Dh, seg, ptr(h0), ptr(ckpt), ptr(dq), ptr(dk), ptr(dv), ptr(dg),
        ptr(dh0), ptr(ws), 0 if ws is None else ws.numel(), stream_of(q))
    _check(rc, "rr_gla_bwd")


# ---------------------------------------------------------------- RG-LRU
def rglru_workspace(B, L, D, seg, dtype, pass_, device) -> torch.Tensor:
    n = _ws_bytes("rr_rglru_workspace_bytes", (B, L, D, seg, DTYPE_CODE[dtype], pass_))
    return torch.empty(n, dtype=torch.uint8, device=device)


def rglru_fwd(a, x, h0, seg, y, ckpt, ws):
    B, L, D = a.shape
    rc = load().rr_rglru_fwd(ptr(a), ptr(x), DTYPE_CODE[a.dtype], B, L, D, seg,
                             ptr(h0), ptr(y), ptr(ckpt), ptr(ws), ws.numel(), stream_of(a))
    _check(rc, "rr_rglru_fwd")


def rglru_bwd(dy, dfinal, a, x, h0, ckpt, seg, da, dx, dh0, ws):
    B, L, D = a.shape
    rc = load().rr_rglru_bwd(ptr(dy), ptr(dfinal), ptr(a), ptr(x), DTYPE_CODE[a.dtype],
                             B, L, D, seg, ptr(h0), ptr(ckpt), ptr(da), ptr(dx), ptr(dh0),
                             ptr(ws), ws.numel(), stream_of(a))
    _check(rc, "rr_rglru_bwd")


def rglru_gated_workspace(B, L, D, seg, dtype, pass_, device) -> torch.Tensor:
    n = _ws_bytes("rr_rglru_gated_workspace_bytes", (B, L, D, seg, DTYPE_CODE[dtype], pass_))
    return torch.empty(n, dtype=torch.uint8, device=device)


def rglru_gated_fwd(r, i, x, lam, c, h0, seg, y, ckpt, ws):
    B, L, D = r.shape
    rc = load().rr_rglru_gated_fwd(ptr(r), ptr(i), ptr(x), ptr(lam), float(c), DTYPE_CODE[r.dtype],
                                   B, L, D, seg, ptr(h0), ptr(y), ptr(ckpt), ptr(ws), ws.numel(),
                                   stream_of(r))
    _check(rc, "rr_rglru_gated_fwd")


def rglru_gated_bwd(dy, dfinal, r, i, x, lam, c, h0, ckpt, seg, dr, di, dx, dlam, dh0, ws):
    B, L, D = r.shape
    rc = load().rr_rglru_gated_bwd(ptr(dy), ptr(dfinal), ptr(r), ptr(i), ptr(x), ptr(lam), float(c),
                                   DTYPE_CODE[r.dtype], B, L, D, seg, ptr(h0), ptr(ckpt), ptr(dr),
                                   ptr(di), ptr(dx), ptr(dlam), ptr(dh0), ptr(ws), ws.numel(),
                                   stream_of(r))
    _check(rc, "rr_rglru_gated_bwd")


# ---------------------------------------------------------------- rotLRU
def rotlru_workspace(B, L, Dp, seg, dtype, pass_, device) -> torch.Tensor:
    n = _ws_bytes("rr_rotlru_workspace_bytes", (B, L, Dp, seg, DTYPE_CODE[dtype], pass_))
    return torch.empty(n, dtype=torch.uint8, device=device)


def rotlru_fwd(a, cs, sn, x, h0, seg, y, ckpt, ws):
    B, L, Dp = a.shape
    rc = load().rr_rotlru_fwd(ptr(a), ptr(cs), ptr(sn), ptr(x), DTYPE_CODE[a.dtype],
                              B, L, Dp, seg, ptr(h0), ptr(y), ptr(ckpt), ptr(ws), ws.numel(), stream_of(a))
    _check(rc, "rr_rotlru_fwd")


def rotlru_bwd(dy, dfinal, a, cs, sn, x, h0, ckpt, seg, da, dcs, dsn, dx, dh0, ws):
    B, L, Dp = a.shape
    rc = load().rr_rotlru_bwd(ptr(dy), ptr(dfinal), ptr(a), ptr(cs), ptr(sn), ptr(x),
                              DTYPE_CODE[a.dtype], B, L, Dp, seg, ptr(h0), ptr(ckpt),
                              ptr(da), ptr(dcs), ptr(dsn), ptr(dx), ptr(dh0), ptr(ws), ws.numel(),
                              stream_of(a))
    _check(rc, "rr_rotlru_bwd")


def rotlru_theta_fwd(a, th, x, h0, seg, y, ckpt, ws):
    B, L, Dp = a.shape
    rc = load().rr_rotlru_theta_fwd(ptr(a), ptr(th), ptr(x), DTYPE_CODE[a.dtype], B, L, Dp, seg,
                                    ptr(h0), ptr(y), ptr(ckpt), ptr(ws), ws.numel(), stream_of(a))
    _check(rc, "rr_rotlru_theta_fwd")


def rotlru_theta_bwd(dy, dfinal, a, th, x, h0, ckpt, seg, da, dth, dx, dh0, ws):
    B, L, Dp = a.shape
    rc = load().rr_rotlru_theta_bwd(ptr(dy), ptr(dfinal), ptr(a), ptr(th), ptr(x), DTYPE_CODE[a.dtype],
                                    B, L, Dp, seg, ptr(h0), ptr(ckpt), ptr(da), ptr(dth), ptr(dx),
                                    ptr(dh0), ptr(ws), ws.numel(), stream_of(a))
    _check(rc, "rr_rotlru_theta_bwd")


# ---------------------------------------------------------------- decode steps
def ssd_step(u, delta, Bm, Cm, A, a_stride_n, state, y):
    B, H, Dh = u.shape
    N = Bm.shape[-1]
    _check(load().rr_ssd_step(ptr(u), ptr(delta), ptr(Bm), ptr(Cm), ptr(A), a_stride_n, DTYPE_CODE[u.dtype],
                              B, H, Dh, N, ptr(state), ptr(y), stream_of(u)), "rr_ssd_step")


def gla_step(q, k, v, g, state, y):
    B, H, Dh = q.shape
    _check(load().rr_gla_step(ptr(q), ptr(k), ptr(v), ptr(g), DTYPE_CODE[q.dtype], B, H, Dh, ptr(state), ptr(y),
                              stream_of(q)), "rr_gla_step")


def rglru_step(a, x, state, y):
    B, D = a.shape
    _check(load().rr_rglru_step(ptr(a), ptr(x), DTYPE_CODE[a.dtype], B, D, ptr(state), ptr(y), stream_of(a)),
           "rr_rglru_step")


def rotlru_step(a, cs, sn, x, state, y):
    B, Dp = a.shape
    _check(load().rr_rotlru_step(ptr(a), ptr(cs), ptr(sn), ptr(x), DTYPE_CODE[a.dtype], B, Dp, ptr(state), ptr(y),
                                 stream_of(a)), "rr_rotlru_step")


# ---------------------------------------------------------------- Gated DeltaNet
def gdn_fwd(q, k, v, alpha, beta, h0, seg, y, ckpt, ws=None):
    """ws: gdn_fwd_workspace(...) for the chunkwise form (None: sequential)."""
    B, L, H, Dh = q.shape
    _check(load().rr_gdn_fwd(ptr(q), ptr(k), ptr(v), ptr(alpha), ptr(beta), DTYPE_CODE[q.dtype], B, L, H, Dh, seg,
                             ptr(h0), ptr(y), ptr(ckpt), ptr(ws), 0 if ws is None else ws.numel(), stream_of(q)),
           "rr_gdn_fwd")


def gdn_fwd_workspace(B, L, H, Dh, seg, dtype, device) -> torch.Tensor | None:
    return _alloc_ws(_ws_bytes("rr_gdn_fwd_workspace_bytes", (B, L, H, Dh, seg, DTYPE_CODE[dtype])), device)


def gdn_workspace(B, L, H, Dh, seg, dtype, device) -> torch.Tensor | None:
    return _alloc_ws(_ws_bytes("rr_gdn_workspace_bytes", (B, L, H, Dh, seg, DTYPE_CODE[dtype])), device)


def gdn_bwd(dy, dfinal, q, k, v, alpha, beta, h0, ckpt, seg, dq, dk, dv, dalpha, dbeta, dh0, ws):
    B, L, H, Dh = q.shape
    _check(load().rr_gdn_bwd(ptr(dy), ptr(dfinal), ptr(q), ptr(k), ptr(v), ptr(alpha), ptr(beta),
                             DTYPE_CODE[q.dtype], B, L, H, Dh, seg, ptr(h0), ptr(ckpt), ptr(dq), ptr(dk), ptr(dv),
                             ptr(dalpha), ptr(dbeta), ptr(dh0), ptr(ws), 0 if ws is None else ws.numel(),
                             stream_of(q)), "rr_gdn_bwd")
