"""The C++ suite (tests/cpp/test_vectorcore.cpp) through the C++ API.

Three builds of it: against libvectorcore.so, and compiled with the
runtime's sources under ASan+UBSan and under TSan (the reference runs its C++
suite under both, README.md:116-117). The sanitizer builds run on the cpu
device (hip unavailable or not, only host code is instrumented); the plain
build also runs on hip on a GPU, including an MLP train step through the C++
API. The binaries are built by vectorcore_amd/build.py (build_cpp_tests).
"""

import os
import subprocess
from pathlib import Path

import pytest

BUILD = Path(__file__).resolve().parents[1] / "vectorcore_amd" / "_build"


def run_suite(variant, devices, timeout=300):
    exe = BUILD / variant / "test_vectorcore"
    if not exe.exists():
        pytest.fail(f"{exe} is not built: run python vectorcore_amd/build.py")
    env = dict(os.environ, VECTORCORE_TEST_DEVICES=devices,
               ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1",
               TSAN_OPTIONS="halt_on_error=1:second_deadlock_stack=1")
    r = subprocess.run([str(exe)], env=env, capture_output=True, text=True, timeout=timeout)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert "[FAIL]" not in out and "runtime error" not in out and "WARNING: ThreadSanitizer" not in out, out[-6000:]
    return out


def test_cpp_suite_on_cpu():
    out = run_suite("bin", "cpu")
    assert "26/26 cases passed" in out


def test_cpp_suite_under_asan_and_ubsan():
    run_suite("asan", "cpu")


def test_cpp_suite_under_tsan():
    out = run_suite("tsan", "cpu")
    assert "[PASS] cpu kernels from several threads at once (cpu)" in out


@pytest.mark.gpu
def test_cpp_suite_on_hip():
    out = run_suite("bin", "cpu,hip")
    assert "hip unavailable" not in out, out[-3000:]
    assert "[PASS] MLP train step on hip against the cpu device (hip)" in out
    assert "[PASS] matmul gradients (hip)" in out
