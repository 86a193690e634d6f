"""The host code (graph builder, lowering, arena planner, executor, run-time
compilation) under AddressSanitizer and UBSan: the plan-only backend tests run in
a child process against the sanitizer build of the library
(`make -C go-darwinml_amd/csrc asan`, which __graft_entry__.build() runs), with
clang's ASan runtime preloaded into python.  Any sanitizer report aborts the
child (UBSan is built without recovery), so a clean exit means none fired."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN_LIB = os.path.join(ROOT, "go-darwinml_amd", "csrc", "_build_asan", "libgomlx_hip_asan.so")
CLANGXX = "/opt/rocm/llvm/bin/clang++"


def _asan_runtime():
    try:
        out = subprocess.run([CLANGXX, "-print-file-name=libclang_rt.asan-x86_64.so"], check=True,
                             capture_output=True, text=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return None
    return out if os.path.isabs(out) and os.path.exists(out) else None


def test_plan_tests_clean_under_asan_ubsan():
    rt = _asan_runtime()
    if not os.path.exists(ASAN_LIB) or rt is None:
        pytest.skip("sanitizer build absent: run `make -C go-darwinml_amd/csrc asan`")
    env = dict(os.environ, LD_PRELOAD=rt, GHIP_LIB_PATH=ASAN_LIB,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_graph_plan.py"),
                        os.path.join(ROOT, "tests", "test_abi.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "passed" in r.stdout and "AddressSanitizer" not in tail and "runtime error" not in tail, tail
