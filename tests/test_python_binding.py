"""Port of the reference's Python-binding tests (reference tests/test_python_binding.py:1-49) to the
`ternixengine_amd` module: the same shapes, seeds, numpy oracle and error cases, with the HIP
implementations in place of the CPU and CUDA ones.

The reference checks every CPU impl at (1,8,8), (5,33,24), (64,256,128) and the CUDA impls at
(128,256,192); here every HIP impl runs all four shapes (the `hip_tiled` impl keeps the reference
tiled kernel's M,N,K % 64 contract, so shapes outside it must raise RuntimeError("HIP error: ..."),
which is how the reference binding reports cuda_tiled's cudaErrorInvalidValue, :62-65)."""
import numpy as np
import pytest

import ternixengine_amd as ternix

HIP_IMPLS = ["hip", "hip_gemv", "hip_gemm", "hip_tiled", "hip_naive"]
SHAPES = [(1, 8, 8), (5, 33, 24), (64, 256, 128), (128, 256, 192)]


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


def test_module_attributes():
    assert ternix.has_cuda is False
    assert isinstance(ternix.has_hip, bool)


@pytest.mark.gpu
@pytest.mark.parametrize("impl", HIP_IMPLS)
@pytest.mark.parametrize("shape", SHAPES)
def test_hip_kernels_match_numpy(impl, shape):
    m, k, n = shape
    a, w = make(*shape, seed=sum(shape))
    packed = ternix.pack_ternary(w)
    if (impl == "hip_tiled" and (m % 64 or k % 64 or n % 64)) or (impl == "hip_gemv" and m > 32):
        with pytest.raises(RuntimeError, match="HIP error"):
            ternix.ternary_matmul(a, packed, impl)
        return
    got = ternix.ternary_matmul(a, packed, impl)
    np.testing.assert_array_equal(got, reference(a, w))


@pytest.mark.gpu
def test_default_impl_matches_numpy():
    a, w = make(128, 256, 192, seed=3)
    np.testing.assert_array_equal(ternix.ternary_matmul(a, ternix.pack_ternary(w)), reference(a, w))


def test_input_validation():
    a, w = make(4, 8, 8, 1)
    with pytest.raises(ValueError):
        ternix.pack_ternary((w * 2).astype(np.int8))          # values outside {-1,0,1}
    with pytest.raises(ValueError):
        ternix.ternary_matmul(a, ternix.pack_ternary(w), "nope")
    with pytest.raises(ValueError):
        ternix.ternary_matmul(a[:, :4], ternix.pack_ternary(w))  # inner dimensions
    with pytest.raises(ValueError):
        ternix.ternary_matmul(a.reshape(-1), ternix.pack_ternary(w))  # ndim
