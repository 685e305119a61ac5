"""The Q8_0 GEMV kernel's short forms of d = amax / 127 and of Rust's round are the
reference's operations bit for bit (ferrum_amd/csrc/fkv_gemv.hip: div127,
round_away): checked here over every f32 input on the CPU, where IEEE f32 multiply,
add, fma and trunc give what the GPU's v_mul/v_add/v_fma/v_trunc give."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div127_and_round_half_away_exhaustive(tmp_path):
    exe = tmp_path / "q8_fastmath_check"
    flags = ["-O2", "-ffp-contract=off"]
    try:
        if " fma " in open("/proc/cpuinfo").read().replace("\n", " "):
            flags.append("-mfma")   # hardware fmaf (libm's is correct too, only slower)
    except OSError:
        pass
    subprocess.run(["gcc", *flags, "-o", str(exe),
                    os.path.join(HERE, "fastmath", "q8_fastmath_check.c"), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.stdout.strip() == "div127 0 round 0", out.stdout
    assert out.returncode == 0
