"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (GPU
sanitizers are not available on the GPU pool; device code is left alone):

* the CPU restatement and the record generator (g++):
  tests/cpp/sanitize_driver.cpp drives every configuration, inclusion mode
  and framing through encode and decode, the generator's corruptions and
  seeded byte mutations;
* the host half of libpetjson, pj_api.cpp (hipcc, host code only):
  tests/cpp/api_sanitize.cpp checks argument validation and the decode
  bounds here; tests/test_gpu_sanitized_api.py runs the same binary (built
  by tests/cpp/build.sh) on the GPU, where it also round-trips records
  through the host entry points (their staging copies).

Any report fails the run."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
PKG = os.path.join(ROOT, "micronaut3-bug_amd")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
INC = ["-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "oracle"), "-I" + os.path.join(PKG, "csrc")]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _run(exe, leaks=True):
    env = dict(os.environ, ASAN_OPTIONS=f"detect_leaks={int(leaks)}:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    return r.stdout


def test_oracle_and_generator_clean_under_asan_ubsan(tmp_path):
    objs = []
    for src, lang in ((os.path.join(ROOT, "oracle", "pj_oracle.c"), ["-x", "c", "-std=c11"]),
                      (os.path.join(PKG, "csrc", "pj_gen.cpp"), ["-std=c++17"]),
                      (os.path.join(CPP, "sanitize_driver.cpp"), ["-std=c++17"])):
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        subprocess.run(["g++", *lang, *SAN, *INC, "-c", src, "-o", obj], check=True)
        objs.append(obj)
    exe = str(tmp_path / "sanitize_driver")
    subprocess.run(["g++", *SAN, *objs, "-pthread", "-o", exe], check=True)
    assert "decodes clean" in _run(exe)


def build_api_sanitized(out_dir):
    """pj_api.cpp and pj_gen.cpp host-sanitized, the kernels as built, and
    the API driver, into one executable (needs the in-tree build's objects)."""
    hflags = ["-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=all",
              "-Xarch_host", "-fno-omit-frame-pointer", "-g", "-O1", "-std=c++17", "--offload-arch=gfx950", *INC]
    objs = []
    for src in (os.path.join(PKG, "csrc", "pj_api.cpp"), os.path.join(PKG, "csrc", "pj_gen.cpp"),
                os.path.join(CPP, "api_sanitize.cpp")):
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        subprocess.run([HIPCC, *hflags, "-c", src, "-o", obj], check=True, capture_output=True)
        objs.append(obj)
    kern = [os.path.join(PKG, "_build", f) for f in ("pj_encode_hip.o", "pj_decode_hip.o", "pj_model_hip.o")]
    if not all(os.path.exists(k) for k in kern):
        pytest.skip("kernel objects missing: run __graft_entry__.build() first")
    exe = os.path.join(out_dir, "api_sanitize")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-fsanitize=address,undefined", "-fno-gpu-sanitize", *objs, *kern,
                    "-pthread", "-o", exe], check=True, capture_output=True)
    return exe


def test_api_host_half_clean_under_asan_ubsan(tmp_path):
    """Without a GPU (this container) the driver checks argument validation
    and the bounds; the HIP runtime's own allocations are not ours, so leak
    detection is off for this binary."""
    exe = build_api_sanitized(str(tmp_path))
    assert "api sanitize ok" in _run(exe, leaks=False)

