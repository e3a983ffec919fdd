"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

A second build of every source instruments the host code (argument checks,
weight upload staging, the safetensors parser, the conv and FeedForward
loaders) with ASan + UBSan, device code unchanged. The host-logic test
modules then run against it in a fresh process that preloads the sanitizer
runtime; any report fails the run (UBSan does not recover, ASan aborts on
its first error). No GPU is needed.
"""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

DRIVER = """
import sys
sys.path[:0] = [{paths}]
import relpos_mhsa as M
lib = M.library({lib!r})
assert lib._name == {lib!r}
import pytest
sys.exit(pytest.main(["-q", "-m", "not gpu", "-p", "no:cacheprovider"] + {tests!r}))
"""

HOST_TESTS = ["test_abi.py", "test_checkpoint.py", "test_conv_module.py"]


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc is needed to build the sanitized library")
def test_host_code_under_asan_and_ubsan():
    sys.path.insert(0, os.path.join(ROOT, "mlx-nemo-rs_amd"))
    import build
    lib = build.build_sanitized(jobs=8)
    nm = shutil.which("nm")
    if nm:  # the host code really is instrumented
        syms = subprocess.run([nm, "-D", lib], capture_output=True, text=True).stdout
        assert "__asan_init" in syms and "__ubsan_handle" in syms
    paths = ", ".join(repr(os.path.join(ROOT, p)) for p in ("tests", "oracle", "mlx-nemo-rs_amd", ""))
    code = DRIVER.format(paths=paths, lib=lib, tests=[os.path.join(HERE, t) for t in HOST_TESTS])
    env = dict(os.environ)
    env["LD_PRELOAD"] = build.sanitizer_runtime()
    # Python and torch themselves are not instrumented: their allocations are
    # not leak-checked, and their operator new/delete pairing is not ours
    env["ASAN_OPTIONS"] = "detect_leaks=0:alloc_dealloc_mismatch=0:detect_odr_violation=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    r = subprocess.run([sys.executable, "-c", code], env=env, cwd=ROOT, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    print(out[-3000:])
    assert "AddressSanitizer" not in out and "runtime error:" not in out
    assert r.returncode == 0 and " passed" in out
