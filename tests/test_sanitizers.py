"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer: the oracle,
the weight-file code and the tokenizer, built by tests/sanitize/Makefile and
driven by tests/sanitize/host_sanitize.cpp (valid and malformed inputs).  Any
sanitizer report makes the driver exit non-zero.  CPU only."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang not present")
def test_host_code_is_clean_under_asan_and_ubsan(tmp_path):
    out = str(tmp_path)
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "sanitize"), f"OUT={out}"], check=True,
                   capture_output=True, timeout=600)
    env = dict(os.environ,
               ASAN_OPTIONS="abort_on_error=0:detect_leaks=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               LSAN_OPTIONS="suppressions=" + os.path.join(ROOT, "tests", "sanitize", "lsan.supp"),
               OMP_NUM_THREADS="4")
    r = subprocess.run([os.path.join(out, "host_sanitize"), out], capture_output=True, text=True, env=env,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "sanitize ok" in r.stdout
    assert "runtime error" not in r.stderr     # UBSan diagnostics
