"""The offline CMake build (CMakeLists.txt: libternix_hip.so, the CPU oracle and the C++ bit-exactness
test under ctest) configures with no network access: no FetchContent, no package downloads."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("cmake") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="cmake or ROCm not available")
def test_cmake_configures_offline():
    with tempfile.TemporaryDirectory() as build:
        r = subprocess.run(["cmake", "-S", ROOT, "-B", build], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
        text = open(os.path.join(ROOT, "CMakeLists.txt")).read()
        assert "include(FetchContent)" not in text and "ExternalProject_Add" not in text
        ctest = open(os.path.join(build, "CTestTestfile.cmake")).read()
        assert "hip_matmul_bit_exact" in ctest
