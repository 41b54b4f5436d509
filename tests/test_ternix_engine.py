"""The drop-in `ternix_engine` module (ternixengine_amd/bindings/ternix_engine.cpp) against the
reference's own binding tests (reference tests/test_python_binding.py:1-49): the same helpers,
shapes, seeds, numpy oracle and error cases, for the reference's CPU impl strings (served by the
reference's CPU kernels, loaded here from oracle/_ref as ternix_core would be linked in a real build)
and for the HIP impl strings.  Also the module's names, defaults and exception types
(reference bindings/python/pybind11_wrapper.cpp:17-98)."""
import ctypes
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libternix_ref.so")
HAVE_REF = os.path.exists(REF_LIB)
if HAVE_REF:  # the reference's ternix_core CPU kernels, made visible before the module resolves them
    ctypes.CDLL(REF_LIB, mode=ctypes.RTLD_GLOBAL)
sys.path.insert(0, os.path.join(ROOT, "ternixengine_amd", "bindings"))
ternix = pytest.importorskip("ternix_engine")

CPU_IMPLS = ["naive", "scalar", "avx2", "avx2_blocked"]
HIP_IMPLS = ["hip", "hip_gemv", "hip_gemm", "hip_tiled", "hip_naive"]


def reference(a, w):
    return a.astype(np.int32) @ w.astype(np.int32)


def make(m, k, n, seed):
    rng = np.random.default_rng(seed)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-1, 2, size=(k, n), dtype=np.int8)
    return a, w


def test_pack_unpack_roundtrip():
    _, w = make(1, 32, 24, 0)
    packed = ternix.pack_ternary(w)
    assert packed.shape == (32, 6) and packed.dtype == np.uint8
    np.testing.assert_array_equal(ternix.unpack_ternary(packed), w)


@pytest.mark.skipif(not HAVE_REF, reason="reference CPU kernels (oracle/_ref) not built")
@pytest.mark.parametrize("impl", CPU_IMPLS)
@pytest.mark.parametrize("shape", [(1, 8, 8), (5, 33, 24), (64, 256, 128)])
def test_cpu_kernels_match_numpy(impl, shape):
    a, w = make(*shape, seed=sum(shape))
    got = ternix.ternary_matmul(a, ternix.pack_ternary(w), impl)
    np.testing.assert_array_equal(got, reference(a, w))


@pytest.mark.skipif(not HAVE_REF, reason="reference CPU kernels (oracle/_ref) not built")
def test_default_impl_is_avx2_blocked():
    a, w = make(5, 33, 24, seed=62)
    packed = ternix.pack_ternary(w)
    np.testing.assert_array_equal(ternix.ternary_matmul(a, packed), ternix.ternary_matmul(a, packed, "avx2_blocked"))
    with pytest.raises(ValueError):  # the AVX2 precondition N % 8 (reference :54)
        ternix.ternary_matmul(a, ternix.pack_ternary(make(5, 33, 12, 1)[1]))


@pytest.mark.gpu
@pytest.mark.parametrize("impl", HIP_IMPLS)
@pytest.mark.parametrize("shape", [(1, 8, 8), (5, 33, 24), (64, 256, 128), (128, 256, 192)])
def test_hip_kernels_match_numpy(impl, shape):
    m, k, n = shape
    a, w = make(*shape, seed=sum(shape))
    packed = ternix.pack_ternary(w)
    if (impl == "hip_tiled" and (m % 64 or k % 64 or n % 64)) or (impl == "hip_gemv" and m > 32):
        # a shape the device entry point rejects: RuntimeError("HIP error: ..."), as the reference's
        # cuda_tiled reports cudaErrorInvalidValue (reference :62-65)
        with pytest.raises(RuntimeError, match="HIP error"):
            ternix.ternary_matmul(a, packed, impl)
        return
    np.testing.assert_array_equal(ternix.ternary_matmul(a, packed, impl), reference(a, w))


def test_module_attributes():
    assert ternix.has_cuda is False
    assert isinstance(ternix.has_hip, bool)
    m = ternix.Model("weights.bin")
    assert (m.vocab_size, m.hidden_size, m.num_layers) == (32000, 4096, 32)
    m.num_layers = 2
    assert m.num_layers == 2


def test_input_validation():
    a, w = make(4, 8, 8, 1)
    with pytest.raises(ValueError):
        ternix.pack_ternary((w * 2).astype(np.int8))          # values outside {-1,0,1}
    with pytest.raises(ValueError):
        ternix.ternary_matmul(a, ternix.pack_ternary(w), "nope")
    with pytest.raises(ValueError):
        ternix.ternary_matmul(a[:, :4], ternix.pack_ternary(w), "hip")   # inner dimensions
    with pytest.raises(ValueError):
        ternix.pack_ternary(w[:, :6])                          # N % 4
    with pytest.raises(ValueError):
        ternix.unpack_ternary(np.zeros(4, np.uint8))           # ndim
    with pytest.raises(ValueError):
        ternix.ternary_matmul(a, ternix.pack_ternary(w), "cuda_tiled")  # no CUDA build: unknown impl
