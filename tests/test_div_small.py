"""The conv decode divides by float reciprocals with one integer correction
(`div_small`, csrc/salt_device.hpp); this compiles the header's function for the host and
checks it against exact division for every dividend below 2^22 (the decode's range)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "spiking-affine-lazy-training_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_div_small_exact_below_2_pow_22(tmp_path):
    exe = tmp_path / "div_small_check"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
                    os.path.join(ROOT, "tests", "native", "div_small_check.hip"), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches" in r.stdout
