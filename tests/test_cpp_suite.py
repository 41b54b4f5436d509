"""The C++ bit-exactness suite (tests/cpp/test_hip_matmul.cpp): libternix_hip.so through
include/ternix/hip_kernels.hpp, the face a C++ caller of the reference's cuda_kernels.cuh switches to.
Built by __graft_entry__.build() (make -C tests/cpp); the GPU run is one process for all cases."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "test_hip_matmul")
CASES = ["PackKnownAnswer", "NaiveMatchesCpu", "TiledMatchesCpu", "TiledRejectsUnsupportedShape",
         "ReferenceCpuShapes", "DecodeAndPrefillShapes", "RaggedAndMisalignedShapes",
         "ExtremeActivationsDoNotOverflow", "GraphReplay", "Tile64LayoutMatchesCpu"]


def _exe():
    if not os.path.exists(EXE):
        subprocess.run(["make", "-C", os.path.dirname(EXE)], check=True)
    return EXE


def test_cpp_suite_links_and_lists():
    """Loads libternix_hip.so and the oracle and lists its cases without touching a GPU."""
    r = subprocess.run([_exe(), "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == CASES


@pytest.mark.gpu
def test_cpp_suite_on_gpu():
    r = subprocess.run([_exe()], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    for c in CASES:
        assert f"[  OK  ] {c}" in r.stdout, c
