"""The host-side checks under AddressSanitizer + UndefinedBehaviorSanitizer.

__graft_entry__.build() also builds the library with its host code
instrumented (qppocr_amd/build.py, sanitize=True; the device code is built as
usual and nothing here touches a GPU).  The tests that drive the C ABI's
host-only paths -- argument and spec refusals, net specs checked before the
device, the plan decoder's validation of malformed plans -- run again in a
child process with that library and the ASan runtime preloaded; any memory
error or undefined behaviour aborts the child."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_LIB = os.path.join(ROOT, "qppocr_amd", "_build", "sanitize", "libqppocr_hip.so")


def _asan_runtime():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def test_host_checks_under_asan_ubsan():
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("no clang ASan runtime in this image")
    if not os.path.exists(SAN_LIB):
        pytest.skip("sanitizer build absent (built by __graft_entry__.build())")
    env = dict(os.environ)
    env.update(QPPOCR_HIP_LIB=SAN_LIB, LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        "-m", "not gpu", "tests/test_plan_host.py", "tests/test_abi.py"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "passed" in r.stdout and "AddressSanitizer" not in tail and "runtime error" not in tail
