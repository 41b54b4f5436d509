"""The kernels the automatic dispatch only falls back to (register-staged skinny kernels, generic
kernels for ragged shapes, 256-column GEMM tiles for small M) stay bit-exact: each switch set runs
tests/fallback_paths_run.py in one child process (the library reads its switches once per process)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SWITCHES = [
    {"TERNIX_SKINNY_WAVE": "0"},                                                     # DMA-staged GEMVs
    {"TERNIX_WAVE_SW": "16"},                                                        # 16-byte wave strips
    {"TERNIX_SKINNY_WAVE": "0", "TERNIX_SKINNY_DMA": "0"},                           # short / fast kernels
    {"TERNIX_SKINNY_WAVE": "0", "TERNIX_SKINNY_DMA": "0", "TERNIX_SKINNY_SHORT": "0"},  # fast kernel only
    {"TERNIX_RAGGED_PAD": "0"},                                                      # generic ragged kernels
    {"TERNIX_GEMM_NARROW": "0"},                                                     # 256-column small-M GEMM
]


@pytest.mark.gpu
@pytest.mark.parametrize("env", SWITCHES, ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()))
def test_fallback_kernels_bit_exact(env):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "fallback_paths_run.py")],
                       env={**os.environ, **env}, capture_output=True, text=True, timeout=240)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
