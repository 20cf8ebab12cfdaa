"""The library's host-side planning and error code under AddressSanitizer
and UndefinedBehaviorSanitizer, CPU only: tests/native/host_check (built
host-only from tests/native/host_check.cpp, the library's planner headers
and csrc/api_common.cpp by tests/native/Makefile, which build() runs) checks
the tile plans of both tile sets over a grid of shapes and CU counts (every
64 x 64 output cell computed exactly once, every kernel tile inside the
grid of mapped tiles) and the C ABI's error messages. Any sanitizer report
aborts the program."""
import os
import pathlib
import subprocess

import pytest

NATIVE = pathlib.Path(__file__).resolve().parent / "native"
BIN = NATIVE / "host_check"


@pytest.fixture(scope="module")
def host_check():
    if not BIN.exists():
        r = subprocess.run(["make", "-C", str(NATIVE), str(BIN)], capture_output=True, text=True)
        if r.returncode != 0:
            pytest.fail(f"host_check did not build:\n{r.stderr[-2000:]}")
    return BIN


def test_planner_and_error_path_under_sanitizers(host_check):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([str(host_check)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, f"host_check failed:\n{r.stdout}\n{r.stderr[-4000:]}"
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
    assert " 0 failures" in r.stdout
