"""Host build of the library's codec helpers checked against the oracle.

The E8M0 block-exponent rule of codec.h (branch-free: it runs per block in
the device activation split) against the oracle's search-based
or_e8m0_exponent, over every 61st non-negative f32 pattern plus every power
of two and its neighbours, for the four format maxima (448, 240, 57344, 6).
`host/e8m0_check all` runs all 2^31 patterns (about 4 minutes).
"""
import os
import subprocess

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def test_e8m0_exponent_matches_oracle(tmp_path, oracle):
    exe = str(tmp_path / "e8m0_check")
    odir = os.path.join(ROOT, "oracle")
    subprocess.check_call(["g++", "-O2", "-std=c++17",
                           "-I" + os.path.join(ROOT, "welvet.cuda_amd", "csrc"),
                           os.path.join(ROOT, "tests", "host", "e8m0_check.cpp"),
                           "-L" + odir, "-loracle", "-Wl,-rpath," + odir, "-o", exe])
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("checked ")
