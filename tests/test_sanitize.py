"""The host C code (qs_params.c, the sample.h layer qs_sampler.c over a device stub) and the
CPU restatement (oracle/) built with AddressSanitizer and UndefinedBehaviorSanitizer and
run through their branches (tests/c/sanitize_host.c).  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CDIR = os.path.join(ROOT, "tests", "c")


def test_host_code_under_sanitizers():
    if not shutil.which("gcc") and not shutil.which("cc"):
        pytest.skip("no C compiler")
    b = subprocess.run(["make", "-B", "-C", CDIR, "sanitize_host"], capture_output=True,
                       text=True)
    if b.returncode != 0 and "fsanitize" in b.stderr:
        pytest.skip("the C compiler lacks the sanitizer runtimes")
    assert b.returncode == 0, b.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([os.path.join(CDIR, "sanitize_host")], capture_output=True, text=True,
                       env=env, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr


def test_ring_clamp_under_sanitizers():
    """The kernels' history ring functions (qs_ring.h) keep every slot they touch inside
    the row's ring for any stored capacity, length, head and stride, and record as
    sample.c:83-92 does on valid state (tests/c/ring_clamp.c)."""
    if not shutil.which("gcc") and not shutil.which("cc"):
        pytest.skip("no C compiler")
    b = subprocess.run(["make", "-B", "-C", CDIR, "ring_clamp"], capture_output=True, text=True)
    if b.returncode != 0 and "fsanitize" in b.stderr:
        pytest.skip("the C compiler lacks the sanitizer runtimes")
    assert b.returncode == 0, b.stderr
    r = subprocess.run([os.path.join(CDIR, "ring_clamp")], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ring checks passed" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr
