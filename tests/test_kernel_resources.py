"""Scratch (spill) budget of every kernel, from the compiler's own resource
remarks (-Rpass-analysis=kernel-resource-usage) on the committed sources.

No kernel may spill to scratch, except two forward instantiations whose spill
sits before and after the chunk loop, not in it: the persistent 8-wave forward
at head dim 128 (40 bytes per lane) and the 4-wave forward at head dim 128 with
blocks 128 / 256 (20 bytes per lane).  A spill that appears anywhere else fails
here, on the CPU, before it costs time on the GPU: the generic dQ at head dim
256 once spilled 92 bytes per lane inside its chunk loop and ran 25 % slower
with identical results, which no parity test can see."""

import os
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "simple-vsa_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
FILES = ["common", "coarse", "fine_fwd", "fine_bwd", "fine_f32", "tiling"]
pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")

# (mangled-name pattern, largest scratch in bytes per lane it may have)
ALLOWED = [
    (re.compile(r"sparse_fwd_pp_kernelI(DF16b|DF16_)Li128E"), 40),
    (re.compile(r"sparse_fwd_kernelI(DF16b|DF16_)Li128ELi(128|256)E"), 20),
]


def _remarks(name, out_dir):
    # the same flags as the library build, device code only
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "--cuda-device-only",
           "-Rpass-analysis=kernel-resource-usage", "-I" + CSRC, "-c",
           os.path.join(CSRC, name + ".hip"), "-o", os.path.join(out_dir, name + ".o")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stderr


@pytest.fixture(scope="module")
def scratch(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("res"))
    with ThreadPoolExecutor(max_workers=len(FILES)) as ex:
        logs = list(ex.map(lambda f: _remarks(f, out), FILES))
    res, cur = {}, None
    for log in logs:
        for ln in log.splitlines():
            m = re.search(r"remark: Function Name: (\S+)", ln)
            if m:
                cur = m.group(1)
                continue
            m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", ln)
            if m and cur:
                res[cur] = int(m.group(1))
    return res


def test_every_kernel_reports_its_resources(scratch):
    kinds = {"sparse_fwd_pp_kernel", "sparse_fwd_kernel", "sparse_dq_pp_kernel",
             "sparse_dq_kernel", "sparse_dkdv_kernel", "bwd_prep_kernel", "pool_qkv_kernel",
             "csr_cols_kernel", "dkdv_order_kernel"}
    seen = {k for k in kinds for n in scratch if k + "I" in n or k + "E" in n}
    assert seen == kinds, kinds - seen
    assert len(scratch) > 150


def test_no_kernel_spills_beyond_its_budget(scratch):
    over = []
    for name, size in scratch.items():
        limit = next((lim for pat, lim in ALLOWED if pat.search(name)), 0)
        if size > limit:
            over.append(f"{name}: {size} B/lane (allowed {limit})")
    assert not over, "\n".join(over)
