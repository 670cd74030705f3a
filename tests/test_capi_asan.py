"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

Every entry point is called with null device pointers and extreme sizes (see
tests/asan_host_driver.py) in a child process that preloads the sanitizer runtime and
loads the host-sanitized build of the library (``build_lib.py --asan``; device code
unchanged). Out-of-bounds host accesses and signed overflow in the size checks abort
that process; every call must instead return a status."""

import os
import subprocess
import sys

import pytest

from conftest import ROOT

PKG = os.path.join(ROOT, "architecture-zarelga-superposition_amd")


def _asan_lib():
    sys.path.insert(0, PKG)
    import build_lib

    if not os.path.exists(build_lib.ASAN_LIB):
        try:
            build_lib.hipcc()
        except RuntimeError:
            pytest.skip("hipcc not available to build the sanitized library")
        build_lib.build(asan=True)
    return build_lib.ASAN_LIB, build_lib.asan_runtime()


def test_c_abi_host_checks_under_sanitizers():
    lib, runtime = _asan_lib()
    env = dict(os.environ, LD_PRELOAD=runtime, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run(
        [sys.executable, os.path.join(ROOT, "tests", "asan_host_driver.py"), lib,
         os.path.join(PKG, "zmoe", "_lib.py"), os.path.join(ROOT, "include", "zmoe.h")],
        env=env, capture_output=True, text=True, timeout=600)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert "no report" in res.stdout
