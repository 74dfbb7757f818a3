"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

build.build_sanitized() rebuilds the host sources (the pool's bookkeeping and host tier, the GGUF
reader, the repacker, the model's host side) with both sanitizers on the host side only, and a child
Python process with the sanitizer runtime preloaded runs the CPU tests that drive that code through
the C ABI: the GGUF reader on hand-built, truncated, corrupted and reference-written files, the
dequantizer, the dry pool (shard planning, acquire / release, exhaustion, pool sizing), the repacker
round trips and the trace replay through the pool. Any sanitizer report fails the child, and so
this test. No GPU call is made.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECKED = ["test_gguf.py", "test_gguf_reference_file.py", "test_dequant.py", "test_pool.py", "test_capi.py",
           "test_trace.py"]


def test_host_code_under_sanitizers(tmp_path):
    from localstack_amd import build
    rt = build.asan_runtime()
    if rt is None:
        pytest.skip("no clang AddressSanitizer runtime under ROCM_PATH")
    lib = build.build_sanitized()
    syms = subprocess.run(["nm", "-D", lib], capture_output=True, text=True).stdout
    assert "__asan_report_load" in syms and "__ubsan_handle_" in syms  # the instrumentation is in
    env = dict(os.environ, LD_PRELOAD=rt, LSTK_LIBRARY=lib,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu"] + \
          [os.path.join(ROOT, "tests", t) for t in CHECKED]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in out
