"""The host runtime's CPU tests (the .pfm loader on valid, corrupt and
hostile files, graph validation, the quantization rewrite) rerun against an
AddressSanitizer + UBSan build of the runtime, in a child process
(pyflamert_amd/csrc/run_sanitized.sh builds it and preloads the sanitizer
runtimes).  Any sanitizer report aborts the child and fails this test."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++ with libasan/libubsan")
def test_runtime_under_asan_ubsan():
    r = subprocess.run([os.path.join(ROOT, "pyflamert_amd", "csrc", "run_sanitized.sh")], cwd=ROOT,
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert " passed" in r.stdout and "failed" not in r.stdout, r.stdout[-2000:]
