"""Register budget of every HIP kernel (CPU: hipcc cross-compiles for gfx950).

A kernel that spills VGPRs to scratch memory runs far slower than its roofline allows (a
runtime argument added to the 256-row GEMM once cost 20 spilled VGPRs and 40 % of its speed), so the
build is checked here: hipcc's kernel-resource-usage remarks must report no spilled VGPRs and no
scratch memory for any kernel in ternixengine_amd/csrc.  Spilled SGPRs are allowed: they are parked
in VGPR lanes (the fused-quantisation skinny kernels hold their per-row scalars that way), which
the zero scratch size confirms.
"""
import concurrent.futures
import os
import re
import shutil
import subprocess

import pytest

from conftest import hip_file_flags

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ternixengine_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def _resources(src):
    cmd = [HIPCC, "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-O3",
           "-std=c++17", "-fPIC", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "--cuda-device-only", "-c",
           "-o", os.devnull, os.path.join(CSRC, src), "-Rpass-analysis=kernel-resource-usage"] + hip_file_flags(src)
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    kernels, name = {}, None
    for line in out.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            kernels[name] = {}
            continue
        m = re.search(r"remark:\s+(VGPRs Spill|SGPRs Spill|ScratchSize \[bytes/lane\]): (\d+)", line)
        if m and name:
            kernels[name][m.group(1)] = int(m.group(2))
    return src, kernels


@pytest.mark.skipif(not (os.path.exists(HIPCC) or shutil.which("hipcc")), reason="hipcc not available")
def test_no_kernel_spills():
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        results = list(ex.map(_resources, SOURCES))
    bad = []
    total = 0
    for src, kernels in results:
        for name, r in kernels.items():
            total += 1
            if r.get("VGPRs Spill", 0) or r.get("ScratchSize [bytes/lane]", 0):
                bad.append((src, name, r))
    assert total > 50, "kernel-resource-usage remarks not found"
    assert not bad, bad
