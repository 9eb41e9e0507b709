"""The product library's host code -- argument validation, workspace and
plan arithmetic, storage binding, launch sequencing -- under AddressSanitizer
and UndefinedBehaviorSanitizer: tests/test_abi.py runs against
_build/asan/libq38m_asan.so (`make asan` in the package directory, which
build() runs: the host code of every source sanitized, the device code the
product's) in a child process with clang's ASan runtime preloaded (its
UBSan handlers included).  Any report aborts the child; leak checking is off
(the interpreter's own allocations would be reported)."""
import os
import subprocess
import sys

import pytest

from conftest import PACKAGE_DIR, ROOT

ASAN_LIB = os.path.join(PACKAGE_DIR, "_build", "asan", "libq38m_asan.so")
CLANG = "/opt/rocm/llvm/bin/clang"

CHILD = r"""
import ctypes, os, sys
import pytest
sys.path.insert(0, os.path.join(sys.argv[1], "tests"))
from conftest import load_product
q38m = load_product()
assert q38m.LIB_PATH == sys.argv[2], q38m.LIB_PATH
assert hasattr(ctypes.CDLL(None), "__asan_init"), "the ASan runtime is not loaded"
sys.exit(pytest.main(["-q", "-x", "-p", "no:cacheprovider",
                      os.path.join(sys.argv[1], "tests", "test_abi.py")]))
"""


def test_abi_under_host_sanitizers():
    if not os.path.exists(ASAN_LIB):
        pytest.fail(f"{ASAN_LIB} is not built; run __graft_entry__.build()")
    if not os.path.exists(CLANG):
        pytest.skip("clang (for its ASan runtime) is not installed")
    runtime = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"],
                             check=True, capture_output=True, text=True).stdout.strip()
    assert os.path.isabs(runtime) and os.path.exists(runtime), runtime
    # the library's host code is instrumented: it calls into both runtimes
    undefined = subprocess.run(["nm", "-D", "--undefined-only", ASAN_LIB], check=True,
                               capture_output=True, text=True).stdout
    assert "__asan_report_load" in undefined and "__ubsan_handle_" in undefined
    env = dict(os.environ, LD_PRELOAD=runtime, Q38M_LIB_PATH=ASAN_LIB,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    child = subprocess.run([sys.executable, "-c", CHILD, ROOT, ASAN_LIB], env=env, cwd=ROOT,
                           capture_output=True, text=True, timeout=600)
    assert child.returncode == 0, child.stdout[-4000:] + child.stderr[-4000:]
    assert " passed" in child.stdout and "failed" not in child.stdout
