"""The C oracle under AddressSanitizer and UndefinedBehaviorSanitizer (CPU
only): `make -C oracle sanitize` builds tfd_oracle.c with a driver
(oracle/sanitize_main.c) that walks its Laya tile/GEMM and scalar paths,
windows, ragged tiles, L = 1, empty inputs, NaN/inf values and short-storage
rejection, and its Jeff paths (GQA expansion, partial and full RoPE, empty
rows), at one and three threads. Any out-of-bounds access, leak or undefined
behaviour aborts the driver."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")


@pytest.mark.skipif(shutil.which("gcc") is None and shutil.which("cc") is None,
                    reason="no C compiler")
def test_oracle_is_clean_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", ORACLE, "sanitize"], check=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([os.path.join(ORACLE, "_build", "sanitize_driver")], capture_output=True,
                       text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "oracle sanitize driver: ok" in r.stdout
