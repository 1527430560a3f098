"""The exact integer helpers of the kernels (taco_amd/csrc/intmath.h), built for the host with
g++ and checked against unsigned __int128 arithmetic and the digit-by-digit square root."""

import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))


def test_intmath_helpers_are_exact():
    src = os.path.join(HERE, "native", "intmath_check.cpp")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "intmath_check")
        subprocess.run(["g++", "-O2", "-std=c++17", "-o", exe, src], check=True)
        out = subprocess.run([exe, "200000"], capture_output=True, text=True, timeout=300)
        assert out.returncode == 0, out.stdout + out.stderr
        assert out.stdout.startswith("ok")
