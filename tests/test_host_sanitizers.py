"""CPU: the library's host code under AddressSanitizer and
UndefinedBehaviorSanitizer.  tests/sanitize/Makefile compiles the C++ shim
and the slot manager with -fsanitize=address,undefined (g++, host code
only), links them with the product's HIP objects and a driver that exercises
the weight-file mapping, the coloured host buffers and their copies, the
layer coordinate, the slot manager, and every entry point's no-device error
path; the driver runs in its own process (the sanitizer runtime must own it)
and any report, leaks included, fails the test."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import pytest

from conftest import ROOT, gncx

SAN_DIR = ROOT / "tests" / "sanitize"


def _gpu_visible() -> bool:
    try:
        hip = C.CDLL("libamdhip64.so")
    except OSError:
        return False
    n = C.c_int(0)
    return hip.hipGetDeviceCount(C.byref(n)) == 0 and n.value > 0


@pytest.mark.skipif(_gpu_visible(), reason="the driver checks the no-device paths; run on a CPU-only host")
def test_host_exports_clean_under_asan_and_ubsan(tmp_path):
    if not all((ROOT / "gnc-x_amd" / "_build" / f"{n}.o").exists()
               for n in ("gemv", "attention", "elementwise", "matbatch", "noalloc")):
        out = subprocess.run(["make", "-C", str(gncx.CSRC_DIR), "-j8"], capture_output=True, text=True)
        assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    build = tmp_path / "build"
    out = subprocess.run(["make", "-C", str(SAN_DIR), f"OUT={build}"], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    run = subprocess.run([str(build / "host_exports_driver"), str(tmp_path)], capture_output=True, text=True,
                         env=env, timeout=300)
    report = run.stdout[-3000:] + run.stderr[-3000:]
    assert run.returncode == 0, report
    assert "clean under the sanitizers" in run.stdout, report
    assert "runtime error" not in run.stderr and "AddressSanitizer" not in run.stderr, report
