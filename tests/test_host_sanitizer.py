"""The C ABI's host-side planning code under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only).

csrc/plan.cpp holds what the entry points decide on the host before any
launch: the Hessian's token splits and workspace runs, the factorisation's
recursion scratch, the sweep workspace, the register-decoded GEMM plan and
split-K rules, every *_workspace_size query and the gptq::linear argument
checks.  It has no HIP dependency, so g++ builds it with
-fsanitize=address,undefined beside tests/host/plan_check.cpp, which walks
those functions over grids of shapes (extreme sizes included), checks their
properties and prints every query's result.  The test requires a clean run
and the same results from the shipped libgptq_hip.so (the same source built
by hipcc)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "distributed_gptq_amd", "csrc")


@pytest.fixture(scope="module")
def sanitized_run(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("host_asan") / "plan_check")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "host", "plan_check.cpp"), os.path.join(CSRC, "plan.cpp"),
           os.path.join(CSRC, "status.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    return r


def test_planning_code_is_clean_under_asan_and_ubsan(sanitized_run):
    r = sanitized_run
    assert "runtime error" not in r.stderr, r.stderr[-2000:]
    assert "AddressSanitizer" not in r.stderr and "LeakSanitizer" not in r.stderr, r.stderr[-2000:]
    assert r.returncode == 0, r.stderr[-2000:]
    assert "0 check(s) failed" in r.stderr
    assert len(r.stdout.splitlines()) > 10000


def test_sanitized_build_agrees_with_the_shipped_library(sanitized_run):
    """Every workspace query the harness printed gives the same value from
    libgptq_hip.so (host-only calls, no GPU needed)."""
    from distributed_gptq_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.load()
    n = 0
    for line in sanitized_run.stdout.splitlines():
        lhs, val = line.split(" = ")
        name, *args = lhs.split()
        got = getattr(lib, name)(*[int(a) for a in args])
        assert got == int(val), (line, got)
        n += 1
    assert n > 10000
