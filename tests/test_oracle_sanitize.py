"""AddressSanitizer / UndefinedBehaviorSanitizer run of the CPU oracle (the
counterpart of the reference's `make test-race`, Makefile:306): every
oracle entry point over edge-case inputs (zero / NaN / inf blocks, ragged
lengths, every row type in both orders, the AVX2 port, a tiny llama with and
without the repeat penalty) with leak checking on.  Host code only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")


def test_oracle_clean_under_asan_ubsan():
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    subprocess.run(["make", "-s", "-C", ORACLE, "-B", "sanitize"], check=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="2")
    r = subprocess.run([os.path.join(ORACLE, "_san", "oracle_sanitize")], env=env,
                       capture_output=True, text=True, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "oracle sanitize: ok" in out
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
