"""Shared fixtures.  The CPU oracle (oracle/liboracle.so) is test infrastructure: only tests, smoke()
and bench.py's cpu_baseline use it, always as the checker."""
import ctypes
import json
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def hip_file_flags(src):
    """Extra hipcc flags the library's Makefile gives one source (the GEMV kernels' kernel-argument
    preload count), so that tests reading the emitted code see what the library runs."""
    if src not in ("line_gemv.hip", "skinny_kernels.hip"):
        return []
    import re
    with open(os.path.join(ROOT, "ternixengine_amd", "csrc", "Makefile")) as f:
        n = re.search(r"^LINE_PRELOAD \?= (\d+)", f.read(), re.M).group(1)
    return ["-mllvm", f"-amdgpu-kernarg-preload-count={n}"]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(autouse=True)
def _no_device_faults(request):
    """Every GPU test ends with the library's device fault word clear: no bounded in-launch wait of
    the kernels gave up during the test (such a wait does not fail the call, it records a bit)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    from ternixengine_amd import _lib
    bits = ctypes.c_uint(0)
    st = _lib.load().ternix_hip_take_faults(ctypes.byref(bits))
    assert st == 0, f"ternix_hip_take_faults failed: {st}"
    assert bits.value == 0, f"device fault word 0x{bits.value:x} after {request.node.nodeid}"


def _oracle_lib():
    so = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "liboracle.so"], check=True)
    lib = ctypes.CDLL(so)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    for n in ("oracle_pack_ternary", "oracle_unpack_ternary", "oracle_interleave"):
        getattr(lib, n).argtypes = [vp, vp, sz]
        getattr(lib, n).restype = None
    for n in ("oracle_mm_naive", "oracle_mm_scalar", "oracle_gemm_unpacked"):
        getattr(lib, n).argtypes = [vp, vp, vp, sz, sz, sz]
        getattr(lib, n).restype = None
    for n in ("oracle_mm_avx2", "oracle_mm_avx2_blocked"):
        getattr(lib, n).argtypes = [vp, vp, vp, sz, sz, sz]
        getattr(lib, n).restype = ctypes.c_int
    lib.oracle_mm_scalar_mt.argtypes = [vp, vp, vp, sz, sz, sz, ctypes.c_int]
    lib.oracle_mm_scalar_mt.restype = None
    return lib


class Oracle:
    """numpy-facing wrapper of the C oracle."""

    def __init__(self):
        self.lib = _oracle_lib()

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(ctypes.c_void_p)

    def pack(self, w):
        w = np.ascontiguousarray(w, dtype=np.int8)
        out = np.empty(w.shape[:-1] + (w.shape[-1] // 4,), np.uint8)
        self.lib.oracle_pack_ternary(self._p(out), self._p(w), w.size)
        return out

    def unpack(self, wp):
        wp = np.ascontiguousarray(wp, dtype=np.uint8)
        out = np.empty(wp.shape[:-1] + (wp.shape[-1] * 4,), np.int8)
        self.lib.oracle_unpack_ternary(self._p(out), self._p(wp), out.size)
        return out

    def mm(self, kind, a, wp, n=None):
        a = np.ascontiguousarray(a, dtype=np.int8)
        wp = np.ascontiguousarray(wp, dtype=np.uint8)
        m, k = a.shape
        n = wp.shape[1] * 4 if n is None else n
        c = np.full((m, n), -999, np.int32)
        if kind == "scalar_mt":
            self.lib.oracle_mm_scalar_mt(self._p(a), self._p(wp), self._p(c), m, k, n, min(16, os.cpu_count() or 1))
        else:
            r = getattr(self.lib, f"oracle_mm_{kind}")(self._p(a), self._p(wp), self._p(c), m, k, n)
            if r not in (None, 0):
                raise ValueError(f"oracle {kind} rejected N={n}")
        return c

    def gemm_unpacked(self, a, w):
        a = np.ascontiguousarray(a, dtype=np.int8)
        w = np.ascontiguousarray(w, dtype=np.int8)
        c = np.empty((a.shape[0], w.shape[1]), np.int32)
        self.lib.oracle_gemm_unpacked(self._p(a), self._p(w), self._p(c), a.shape[0], a.shape[1], w.shape[1])
        return c


@pytest.fixture(scope="session")
def oracle():
    return Oracle()


@pytest.fixture(scope="session")
def golden():
    with np.load(os.path.join(GOLDEN, "small_cases.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def digests():
    with open(os.path.join(GOLDEN, "config_digests.json")) as f:
        return json.load(f)["cases"]


def small_case_list(golden):
    return [tuple(int(x) for x in golden[f"s{i}_shape"]) + (i,) for i in range(int(golden["n_small"]))]
