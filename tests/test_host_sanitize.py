"""The C ABI's host code under AddressSanitizer + UndefinedBehaviorSanitizer —
CPU only.

The CPU tests of the C ABI (argument validation and its error texts,
workspace sizing, the tile schedule, the workspace bound walk) run again, in a
child process, against the host-sanitizer build of the library
(`python mlx-recurrence_amd/build.py --host-sanitize`, made by
`__graft_entry__.build()`) with the ASan runtime preloaded; any sanitizer
report ends that process with an error.
"""
import importlib.util
import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
SAN_LIB = ROOT / "mlx-recurrence_amd" / "_build" / "sanitize" / "librecurrence_gfx950.so"
TESTS = ["tests/test_abi.py", "tests/test_tile_schedule.py", "tests/test_workspace_bounds.py",
         "tests/test_host_api.py"]


def _asan_runtime():
    spec = importlib.util.spec_from_file_location("rr_build", ROOT / "mlx-recurrence_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.asan_runtime()


@pytest.mark.skipif(not SAN_LIB.exists(), reason="host-sanitizer build absent "
                    "(python mlx-recurrence_amd/build.py --host-sanitize)")
def test_c_abi_host_code_under_asan_and_ubsan():
    env = dict(os.environ)
    env.update(LD_PRELOAD=str(_asan_runtime()), MLX_RECURRENCE_AMD_LIB=str(SAN_LIB),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *TESTS],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = (res.stdout + res.stderr)[-3000:]
    assert res.returncode == 0, tail
    assert "AddressSanitizer" not in tail and "runtime error" not in tail, tail
    assert " passed" in tail


def test_sanitized_library_is_instrumented():
    if not SAN_LIB.exists():
        pytest.skip("host-sanitizer build absent")
    syms = subprocess.run(["nm", "-D", str(SAN_LIB)], capture_output=True, text=True).stdout
    assert "__asan_report" in syms and "__ubsan_handle" in syms
