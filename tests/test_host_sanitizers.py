"""Host AddressSanitizer + UndefinedBehaviorSanitizer run of the host C++.

The reference builds its runtime, backends and C++ tests under
-fsanitize=address,undefined (CMakeLists.txt:51-69) and its CI runs them
(.github/workflows/ci.yml:173-175). Here tests/cpp/sanitize.mk builds, with
the same sanitizers and leak detection:

* pool_host_test: the bounded pool of the C ABI runtime (runtime.hip) through
  its injectable allocator, on one thread and on eight;
* hip_backend_contract: core/*.cpp and HipBackend::execute rejecting malformed
  requests before any allocation, with a pool over a host allocator (exit 77:
  no device here);
* device_interval_test: the profiling session and the device-interval event
  seam;
* launch_grid_test: the launch grid arithmetic;
* oracle_kat_test: the CPU oracle on known answers, one and four threads.

Each must finish with no sanitizer report. A last test plants a heap overflow
and a signed overflow in a program of its own to show that the build reports
them. No device is used: this runs in the CPU suite.
"""

from __future__ import annotations

import os
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
MAKEFILE = ROOT / "tests" / "cpp" / "sanitize.mk"
CLANG = pathlib.Path("/opt/rocm/llvm/bin/clang++")
ENV = {
    **os.environ,
    "ASAN_OPTIONS": "detect_leaks=1:halt_on_error=1:detect_stack_use_after_return=1:strict_string_checks=1",
    "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
}
ENV.pop("TENSORCX_REQUIRE_HIP", None)
REPORTS = ("ERROR: AddressSanitizer", "ERROR: LeakSanitizer", "runtime error:")

PROGRAMS = {
    "pool_host_test": (0, "pool host test passed"),
    "oracle_kat_test": (0, "oracle known-answer test passed"),
    "device_interval_test": (0, "ok (0 failures)"),
    "launch_grid_test": (0, "ok (0 failures)"),
    "hip_backend_contract": (77, "malformed requests rejected before allocation"),
}


@pytest.fixture(scope="module")
def sanitized(tmp_path_factory):
    if not CLANG.exists() or shutil.which("make") is None:
        pytest.skip("ROCm clang++ or make is missing")
    if not list((ROOT / "tensor.cx_amd" / "_build").glob("gemm.o")):
        pytest.fail("the kernel objects are not built: run `python tensor.cx_amd/build.py`")
    out = tmp_path_factory.mktemp("sanitized")
    result = subprocess.run(["make", "-f", str(MAKEFILE), f"OUT={out}", "-j8"], capture_output=True, text=True,
                            timeout=600)
    assert result.returncode == 0, result.stdout[-4000:] + result.stderr[-4000:]
    return out


@pytest.mark.parametrize("name", sorted(PROGRAMS))
def test_program_is_clean_under_asan_ubsan(sanitized, name):
    from conftest import gpu_present
    if name == "hip_backend_contract" and gpu_present():
        pytest.skip("a device is present: the contract's device part runs in tests/test_hip_contract.py")
    code, marker = PROGRAMS[name]
    result = subprocess.run([str(sanitized / name)], capture_output=True, text=True, timeout=300, env=ENV)
    output = result.stdout + result.stderr
    assert not any(r in output for r in REPORTS), output[-6000:]
    assert result.returncode == code, output[-6000:]
    assert marker in output


PLANTED = r"""
#include <climits>
#include <cstdio>
#include <cstdlib>
int main(int argc, char** argv) {
  int* p = static_cast<int*>(std::malloc(4 * sizeof(int)));
  if (argv[1][0] == 'h') p[argc + 3] = 1;                       // one past the end
  if (argv[1][0] == 'u') { volatile int big = INT_MAX; std::printf("%d\n", big + argc); }  // signed overflow
  std::free(p);
  return 0;
}
"""


@pytest.mark.parametrize("mode,report", [("heap", "heap-buffer-overflow"), ("ub", "signed integer overflow")])
def test_planted_mistakes_are_reported(sanitized, tmp_path, mode, report):
    line = subprocess.run(["make", "-s", "-f", str(MAKEFILE), "print-cxx"], capture_output=True, text=True,
                          check=True).stdout.split()
    src = tmp_path / "planted.cpp"
    src.write_text(PLANTED)
    exe = tmp_path / "planted"
    compiler, flags = line[0], line[1:]
    subprocess.run([compiler, *flags, str(src), "-o", str(exe)], check=True, capture_output=True)
    result = subprocess.run([str(exe), mode], capture_output=True, text=True, timeout=60, env=ENV)
    assert result.returncode != 0
    assert report in result.stderr, result.stderr[-3000:]
