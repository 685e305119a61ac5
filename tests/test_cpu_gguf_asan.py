"""CPU: the GGUF reader's host code under AddressSanitizer and UBSan.

tests/asan/gguf_fuzz.cpp is built with g++ together with ferrum_amd/csrc/fkv_gguf.cpp
(-fsanitize=address,undefined, no recovery) and run over 5,000 seeded mutations of the
rich file of test_cpu_gguf.py (truncations, byte flips, 8- and 4-byte field overwrites,
insertions). Every accepted file is read through info, tensor, find, meta, array
elements and dump. Any sanitizer report fails the run. Skipped where g++ or the HIP
runtime library is missing.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def test_gguf_reader_mutations_under_asan(tmp_path):
    from tests.test_cpu_gguf import _rich
    gxx = shutil.which("g++")
    if gxx is None or not os.path.exists(os.path.join(ROCM, "lib", "libamdhip64.so")):
        pytest.skip("g++ or libamdhip64 missing")
    exe = str(tmp_path / "gguf_fuzz")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
           "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROCM, "include"),
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "ferrum_amd", "csrc"),
           os.path.join(ROOT, "tests", "asan", "gguf_fuzz.cpp"),
           os.path.join(ROOT, "ferrum_amd", "csrc", "fkv_gguf.cpp"), "-o", exe,
           "-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib"),
           "-lpthread"]
    b = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if b.returncode != 0 and "sanitizer" in (b.stderr or "").lower():
        pytest.skip("sanitizer runtime missing: " + b.stderr[-300:])
    assert b.returncode == 0, b.stderr[-2000:]
    seed = tmp_path / "seed.gguf"
    seed.write_bytes(_rich())
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, str(seed), "5000", "12345", str(tmp_path / "case.gguf")],
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, (r.stdout[-1000:], r.stderr[-3000:])
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    ok = int(r.stdout.split("ok ")[1].split()[0])
    err = int(r.stdout.split("err ")[1].split()[0])
    assert ok >= 500 and err >= 500, r.stdout
