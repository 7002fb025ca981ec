"""Build librecurrence_gfx950.so from csrc/*.hip with hipcc (AOT, gfx950 only),
then the C++ autograd bindings (csrc_torch/autograd.cpp -> the Python module
mlx_recurrence_amd._autograd, linked against that library).

Usage:  python mlx-recurrence_amd/build.py [--jobs N] [--verbose] [--host-sanitize]

Objects go to mlx-recurrence_amd/_build/; the shared libraries are written next
to the Python package (mlx_recurrence_amd/), where the loaders look for them.
Every call recompiles (the build check must see the current sources).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
PKG = HERE / "mlx_recurrence_amd"
LIB_NAME = "librecurrence_gfx950.so"
EXT_SRC = HERE / "csrc_torch" / "autograd.cpp"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from forming packed fp32 ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
]


# Host-sanitizer build (--host-sanitize): the host side of the C ABI
# (argument validation, workspace sizing, the tile schedule and workspace
# bound walks) under AddressSanitizer + UndefinedBehaviorSanitizer, for the
# CPU tests.  Only host code is instrumented (each -fsanitize= behind
# -Xarch_host); the device code is built unoptimised, since this library never
# launches a kernel.  Loaded by setting MLX_RECURRENCE_AMD_LIB to its path with
# the ASan runtime preloaded (tests/test_host_sanitize.py).
SANITIZE_DIR = BUILD / "sanitize"
SANITIZERS = ("address", "undefined")
SANITIZE_LINK = [arg for name in SANITIZERS for arg in ("-Xarch_host", "-fsanitize=" + name)]
SANITIZE_FLAGS = [
    f"--offload-arch={ARCH}", "-O1", "-g", "-std=c++17", "-fPIC", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    *SANITIZE_LINK, "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_device", "-O0",
]


def asan_runtime() -> pathlib.Path:
    """The clang ASan runtime that a host-sanitizer build needs preloaded."""
    root = pathlib.Path(hipcc()).resolve().parents[1] / "llvm" / "lib" / "clang"
    for cand in sorted(root.glob("*/lib/linux/libclang_rt.asan-x86_64.so"), reverse=True):
        return cand
    raise RuntimeError(f"libclang_rt.asan-x86_64.so not found under {root}")


def build_sanitized(jobs: int | None = None, verbose: bool = False) -> pathlib.Path:
    SANITIZE_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 8)

    def one(src: pathlib.Path) -> pathlib.Path:
        obj = SANITIZE_DIR / (src.stem + ".o")
        cmd = [hipcc(), *SANITIZE_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"compiling {src.name} (host sanitizers) failed:\n{res.stdout}\n{res.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(one, sources))
    out = SANITIZE_DIR / LIB_NAME
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *SANITIZE_LINK, *map(str, objs), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking the host-sanitizer {LIB_NAME} failed:\n{res.stdout}\n{res.stderr}")
    return out


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (needs ROCm)")


def _compile(src: pathlib.Path, verbose: bool) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    out = PKG / LIB_NAME
    tmp = PKG / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking {LIB_NAME} failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    build_autograd(verbose)
    return out


def build_autograd(verbose: bool = False) -> pathlib.Path:
    """The torch C++ extension mlx_recurrence_amd._autograd (host code only,
    g++ against the installed torch; links librecurrence_gfx950.so by rpath)."""
    import sysconfig

    import torch

    tdir = pathlib.Path(torch.__file__).resolve().parent
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG / ("_autograd" + suffix)
    tmp = PKG / ("_autograd" + suffix + ".tmp")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_autograd",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-isystem", str(tdir / "include"), "-isystem", str(tdir / "include" / "torch" / "csrc" / "api" / "include"),
        "-isystem", "/opt/rocm/include", "-isystem", sysconfig.get_paths()["include"],
        str(EXT_SRC), "-o", str(tmp),
        "-L", str(tdir / "lib"), "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
        "-L", str(PKG), "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the autograd bindings failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--host-sanitize", action="store_true",
                    help="build only the host-sanitizer library (_build/sanitize/) for the CPU tests")
    args = ap.parse_args()
    if args.host_sanitize:
        print(build_sanitized(args.jobs, args.verbose))
    else:
        print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
