"""The device memory helpers of pj_device.h (tile copy-out, LDS and global
byte copies, aligned tail loads, the byte-stream sinks) compiled for the host
and run under AddressSanitizer and UndefinedBehaviorSanitizer with every
buffer sized to exactly what each helper documents, plus PROT_NONE guard
pages around ld_tail's bytes (tests/cpp/device_helpers_check.cpp).  The
unaligned accesses are intended (gfx950 runs global memory in unaligned
mode), so UBSan's alignment check is off."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def test_device_helpers_bounds_under_asan(tmp_path):
    exe = str(tmp_path / "device_helpers_check")
    subprocess.run([HIPCC, "--offload-host-only", "--offload-arch=gfx950", "-std=c++17", "-g", "-O1",
                    "-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize=alignment",
                    "-Xarch_host", "-fno-sanitize-recover=all",
                    "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "micronaut3-bug_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cpp", "device_helpers_check.cpp"), "-o", exe],
                   check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout


def test_decode_block_span_guard(tmp_path):
    """Lines of 4 GiB or more in one decode block are refused (the offsets
    inside a block are 32-bit): tests/cpp/span_guard_check.cpp."""
    exe = str(tmp_path / "span_guard_check")
    subprocess.run([HIPCC, "--offload-host-only", "--offload-arch=gfx950", "-std=c++17", "-g", "-O1",
                    "-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=all",
                    "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "micronaut3-bug_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cpp", "span_guard_check.cpp"), "-o", exe],
                   check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "span guard checks passed" in r.stdout
