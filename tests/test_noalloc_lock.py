"""The lock that serialises pj_encode_device_noalloc calls on one GPU
(micronaut3-bug_amd/csrc/pj_host_lock.h), checked on the host with three
threads (tests/cpp/noalloc_lock_check.cpp): no kernel runs."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_noalloc_calls_on_one_device_serialise(tmp_path):
    exe = str(tmp_path / "noalloc_lock_check")
    subprocess.run(["g++", "-std=c++17", "-O1", "-pthread", "-I", os.path.join(ROOT, "micronaut3-bug_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cpp", "noalloc_lock_check.cpp"), "-o", exe],
                   check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "noalloc lock checks passed" in r.stdout


def test_noalloc_entry_point_takes_the_lock():
    src = open(os.path.join(ROOT, "micronaut3-bug_amd", "csrc", "pj_api.cpp")).read()
    assert "pj::noalloc_lock(ctx->device)" in src
