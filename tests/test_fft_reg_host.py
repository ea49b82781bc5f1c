"""The in-register DFTs of cssm_amd/csrc/fft_reg.h (every FFT pass of the scan and
transform kernels runs them) against a brute-force double-precision DFT, on the host:
tests/fft_reg_check.hip is built with hipcc for the host only and run; no GPU."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_register_dfts_match_bruteforce(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = str(tmp_path / "fft_reg_check")
    subprocess.run([hipcc, "-O2", "-std=c++17", "--cuda-host-only", "-I", os.path.join(ROOT, "cssm_amd", "csrc"),
                    "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "fft_reg_check.hip"),
                    "-o", exe], check=True, capture_output=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")
    rows = [line.split() for line in out if line.strip()]
    assert [(int(n), int(inv)) for n, inv, _ in rows] == [(n, i) for n in (2, 4, 8, 16, 32) for i in (0, 1)]
    for n, inv, err in rows:
        # fp32 rounding of an N-point transform: a few 1e-7 of the output RMS
        assert float(err) <= 1e-6, (n, inv, err)
