"""The host half of libpetjson (pj_api.cpp) in its host-sanitized build
(AddressSanitizer / UndefinedBehaviorSanitizer on host code only; made by
tests/cpp/build.sh) on the GPU: round trips of generated records (configs
1, 3, 5, both framings) through pj_encode_host / pj_decode_host /
pj_decode_array_host and a capacity one short, with any report failing."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "bin", "api_sanitize")

pytestmark = pytest.mark.gpu


def test_api_host_half_clean_sanitized_gpu():
    if not os.path.exists(EXE):
        pytest.skip("tests/cpp/build.sh has not built the sanitized driver")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([EXE], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert "api sanitize ok (gpu)" in r.stdout
