"""The epilogues fold the pooled gradient as x / count with a reciprocal
product and one FMA residual correction (div_by_count in
simple-vsa_amd/csrc/vsa_device.h) instead of a full division per value.  This
host test compiles tests/div_by_count_check.c with gcc and checks that the two
agree bit for bit for every finite bf16 x, every finite fp16 x and every count
in [1, 1024], the domain the kernels use (x is a bf16 or fp16 pooled gradient,
count a block's valid token count)."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_corrected_reciprocal_matches_division(tmp_path):
    exe = tmp_path / "div_by_count_check"
    subprocess.run(["gcc", "-O2", "-mfma", "-o", str(exe), os.path.join(HERE, "div_by_count_check.c"),
                    "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert "bf16 checked" in res.stdout and "fp16 checked" in res.stdout
    assert res.stdout.count("mismatches 0") == 2
