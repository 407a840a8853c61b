"""CPU check of the dK/dV kernel's LDS map and stage protocol.

tests/dkdv_layout_check.hip is a host program built from the kernel's own
configuration (simple-vsa_amd/csrc/dkdv_cfg.h) and swizzle functions: it checks
every (head_dim, block) instantiation's LDS budget and layout, that the
direct-load pieces fill each stage tile exactly where the swizzled reads look,
and replays each step schedule to show that no stage is read before its item
is published or overwritten while it may still be read.  Each planted protocol
mistake must make it fail."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"
SRC = os.path.join(ROOT, "tests", "dkdv_layout_check.hip")
pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")


def _run(tmp_path, define=None):
    exe = tmp_path / ("check_" + (define or "ok"))
    cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-std=c++17",
           "-I" + os.path.join(ROOT, "simple-vsa_amd", "csrc"), SRC, "-o", str(exe)]
    if define:
        cmd.insert(1, "-D" + define)
    subprocess.run(cmd, check=True, capture_output=True)
    return subprocess.run([str(exe)], capture_output=True, text=True)


def test_every_instantiation_passes(tmp_path):
    r = _run(tmp_path)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip().endswith("ALL OK")
    assert r.stdout.count(": ok") == 9, r.stdout


@pytest.mark.parametrize("plant", ["PLANT_SHORT_WAIT", "PLANT_COPY_INTO_READ_STAGE",
                                   "PLANT_LATE_COPY", "PLANT_SWIZZLE"])
def test_planted_protocol_mistakes_fail(tmp_path, plant):
    r = _run(tmp_path, plant)
    assert r.returncode != 0, (plant, r.stdout)
    assert "FAIL" in r.stdout
