"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

* The CPU restatement (oracle/circatt_oracle.c) is built with
  `make -C oracle sanitize` and driven by oracle/sanitize_main.c over small
  shapes, windows wider than the signal included; the driver checks
  invariants (pattern ranges, Distance(x, x) = 0 on the own pixel, Dot
  symmetry, softmax row sums, A ⊗ 1 = rowsum, Aᵀ ⊗ 1 = colsum).
* libcircatt's host code (the C ABI's argument checks and workspace
  arithmetic) is rebuilt with the sanitizers by build.build_host_sanitized and
  the ABI tests (tests/test_abi.py) run against that copy in a child process
  that preloads the sanitizer runtime.  No kernel runs.
"""
import os
import shutil
import subprocess
import sys

import pytest

from conftest import ROOT

PKG = os.path.join(ROOT, "circulantattention.jl_amd")


def test_oracle_under_sanitizers():
    if shutil.which("make") is None or shutil.which("gcc") is None:
        pytest.skip("make / gcc not available")
    oracle = os.path.join(ROOT, "oracle")
    subprocess.run(["make", "-s", "-C", oracle, "sanitize"], check=True, capture_output=True)
    res = subprocess.run([os.path.join(oracle, "_build", "oracle_sanitized")],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all checks passed" in res.stdout


def test_abi_under_sanitizers(tmp_path):
    sys.path.insert(0, PKG)
    import build as B

    if not os.path.exists(B.HIPCC):
        pytest.skip("hipcc not available")
    if not all(os.path.exists(os.path.join(B.OBJ, os.path.splitext(s)[0] + ".o"))
               for s in B.SOURCES if s != "api.cpp"):
        pytest.skip("in-tree objects not built (run build() first)")
    lib = B.build_host_sanitized(str(tmp_path))
    env = dict(os.environ, CIRCATT_LIB=lib, LD_PRELOAD=B.asan_runtime(),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                          os.path.join(ROOT, "tests", "test_abi.py")],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    # the child loaded the instrumented copy
    probe = subprocess.run([sys.executable, "-c",
                            "import sys; sys.path.insert(0, %r); "
                            "from circulant_attention import _lib; print(_lib.LIB_PATH)" % PKG],
                           cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert probe.stdout.strip() == lib, probe.stdout + probe.stderr
