"""The host-side file parsers (GGUF reader, .hos capsule reader) under AddressSanitizer and
UndefinedBehaviorSanitizer: the CPU parser tests — including the reference's fuzz cases
(tests/fuzz_gguf.rs:64-88) and the capsule fuzz — run in a child python against the sanitized build of the
library (`python -m hos_amd.build --sanitize`, host code instrumented, device code as usual). Any report
aborts the child. Skipped when the sanitized build is absent (it takes minutes to build, so build() does not
make it) or older than a source of the library (rebuild it after a change)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_parsers_clean_under_asan_ubsan():
    from hos_amd import build as hb
    if not os.path.exists(hb.SAN_LIB):
        pytest.skip("sanitized library not built (python -m hos_amd.build --sanitize)")
    csrc = os.path.join(ROOT, "hos_amd", "csrc")
    srcs = [os.path.join(csrc, f) for f in os.listdir(csrc)] + [os.path.join(ROOT, "include", "hos_hip.h")]
    if max(os.path.getmtime(f) for f in srcs) > os.path.getmtime(hb.SAN_LIB):
        pytest.skip("sanitized library older than its sources (python -m hos_amd.build --sanitize)")
    rt = hb.asan_runtime()
    assert os.path.exists(rt), rt
    env = dict(os.environ, HOS_HIP_LIB=hb.SAN_LIB, LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_gguf_loader.py"),
                        os.path.join(ROOT, "tests", "test_hos_format.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "passed" in r.stdout and "ERROR: AddressSanitizer" not in r.stderr
    assert "runtime error" not in r.stderr
