"""The host-side C-ABI layer (argument validation, launch configuration, the
scratch-array setup of the allocation-free entry point) under
AddressSanitizer and UndefinedBehaviorSanitizer.

build(sanitize=True) links libdsa_amd_san.so: the product's kernel objects
with the host ABI sources compiled with -fsanitize=address,undefined (host
pass only).  The CPU ABI tests -- every validation path, struct layouts,
exports, size queries -- run against it in a child process with the ASan
runtime preloaded; any report aborts the run.  No GPU is needed: these paths
return before anything is launched.
"""
import os
import subprocess
import sys

import pytest

from dsa_amd import build as hip_build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_abi_tests_pass_under_asan_and_ubsan():
    if not os.path.exists(hip_build.SAN_LIB_PATH):
        hip_build.build(sanitize=True)
    undef = subprocess.run(["nm", "-D", "--undefined-only", hip_build.SAN_LIB_PATH],
                           stdout=subprocess.PIPE, text=True).stdout
    assert "__asan_report" in undef and "__ubsan_handle" in undef, "library is not instrumented"
    runtime = hip_build.sanitizer_runtime()
    assert os.path.exists(runtime), runtime
    env = dict(os.environ, LD_PRELOAD=runtime, DSA_AMD_LIB=hip_build.SAN_LIB_PATH,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
           os.path.join(ROOT, "tests", "test_abi.py"), os.path.join(ROOT, "tests", "test_zz_no_alloc.py")]
    res = subprocess.run(cmd, cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                         text=True, timeout=600)
    tail = "\n".join(res.stdout.splitlines()[-25:])
    assert res.returncode == 0, f"sanitized ABI tests failed:\n{tail}"
    assert "ERROR: AddressSanitizer" not in res.stdout and "runtime error" not in res.stdout, tail
    assert " passed" in tail, tail
