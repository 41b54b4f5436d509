"""CPU-side checks of the product library: it loads, exports every C symbol its headers declare,
validates arguments before touching pointers, and its host code (bitpack, synthetic generators)
matches the oracle.  No kernel is launched here."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

from conftest import ROOT

import ternixengine_amd as tx
from ternixengine_amd import _lib, configs


def declared_c_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "ternix", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"\b(ternix_[a-z0-9_]+)\s*\(", src):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_c_functions()
    assert "ternix_hip_mul_mat_ternary" in names and len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_version():
    assert _lib.load().ternix_hip_version() >= 100


NULL = None


@pytest.mark.parametrize("fn", ["ternix_hip_mul_mat_ternary", "ternix_hip_mul_mat_ternary_gemv",
                                "ternix_hip_mul_mat_ternary_gemm", "ternix_hip_mul_mat_ternary_naive",
                                "ternix_hip_mul_mat_ternary_tiled"])
def test_invalid_shapes_rejected_before_pointer_use(fn):
    f = getattr(_lib.load(), fn)
    assert f(NULL, NULL, NULL, 4, 8, 6, NULL) == 1        # N % 4 != 0
    assert f(NULL, NULL, NULL, -1, 8, 8, NULL) == 1
    assert f(NULL, NULL, NULL, 4, -8, 8, NULL) == 1
    assert f(NULL, NULL, NULL, 4, 8, 1 << 40, NULL) == 1
    if fn != "ternix_hip_mul_mat_ternary_tiled":
        assert f(NULL, NULL, NULL, 4, 8, 8, NULL) == 1    # valid shape, null pointers
        assert f(NULL, NULL, NULL, 0, 8, 8, NULL) == 0    # nothing to do
        assert f(NULL, NULL, NULL, 3, 8, 0, NULL) == 0


def test_tiled_keeps_reference_contract():
    # reference tests/test_cuda_matmul.cu:41-43: (65, 64, 64) rejected with null pointers.
    f = _lib.load().ternix_hip_mul_mat_ternary_tiled
    assert f(NULL, NULL, NULL, 65, 64, 64, NULL) == 1
    assert f(NULL, NULL, NULL, 64, 64, 65 * 4, NULL) == 1
    assert f(NULL, NULL, NULL, 64, 96, 64, NULL) == 1


def test_gemv_rejects_large_m():
    assert _lib.load().ternix_hip_mul_mat_ternary_gemv(NULL, NULL, NULL, 33, 64, 64, NULL) == 1


def test_host_wrapper_validation():
    f = _lib.load().ternix_hip_mul_mat_ternary_host
    assert f(NULL, NULL, NULL, 4, 8, 6, 0) == 1
    assert f(NULL, NULL, NULL, 0, 8, 8, 0) == 0
    a = np.zeros((2, 8), np.int8)
    wp = np.zeros((8, 2), np.uint8)
    c = np.zeros((2, 8), np.int32)
    p = lambda x: x.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    assert f(p(a), p(wp), p(c), 2, 8, 8, 7) == 1          # unknown variant
    assert f(p(a), p(wp), p(c), 33, 8, 8, 2) == 1         # gemv with M > 32
    assert f(p(a), p(wp), p(c), 2, 8, 8, 4) == 1          # tiled contract


def test_error_string():
    assert "invalid" in tx.ternix_error(1).lower()


def test_python_api_validation():
    a = np.zeros((4, 8), np.int8)
    w = np.zeros((8, 8), np.int8)
    with pytest.raises(ValueError):
        tx.pack_ternary((np.ones((8, 8)) * 2).astype(np.int8))
    with pytest.raises(ValueError):
        tx.pack_ternary(np.zeros((8, 6), np.int8))
    with pytest.raises(ValueError):
        tx.pack_ternary(np.zeros(8, np.int8))
    with pytest.raises(ValueError):
        tx.ternary_matmul(a, tx.pack_ternary(w), "nope")
    with pytest.raises(ValueError):
        tx.ternary_matmul(a, tx.pack_ternary(np.zeros((7, 8), np.int8)))
    with pytest.raises(ValueError):
        tx.ternary_matmul(a.ravel(), tx.pack_ternary(w))


def test_pack_matches_oracle_and_reference_bytes(oracle, golden):
    rng = np.random.default_rng(1)
    w = rng.integers(-1, 2, size=(37, 64), dtype=np.int8)
    assert (tx.pack_ternary(w) == oracle.pack(w)).all()
    assert (tx.unpack_ternary(tx.pack_ternary(w)) == w).all()
    assert (tx.pack_ternary(golden["pack_in"].reshape(1, 8)).ravel() == golden["pack_out"]).all()
    allbytes = golden["invalid_Wp"]
    assert (tx.unpack_ternary(allbytes) == golden["invalid_unpacked"]).all()
    for i in range(int(golden["n_small"])):
        assert (tx.pack_ternary(golden[f"s{i}_W"]) == golden[f"s{i}_Wp"]).all()


def test_interleave_is_identity():
    lib = _lib.load()
    src = np.arange(64, dtype=np.uint8)
    dst = np.zeros(64, np.uint8)
    lib.ternix_interleave_weights_offline(dst.ctypes.data_as(ctypes.c_void_p), src.ctypes.data_as(ctypes.c_void_p),
                                          256)
    assert (dst == src).all()


def test_synth_is_deterministic_and_slices_agree():
    lib = _lib.load()
    assert lib.ternix_synth_u64(0, 0, 0) == lib.ternix_synth_u64(0, 0, 0)
    case = configs.CASES["cfg1"]
    a1, a2 = configs.gen_a(case), configs.gen_a(case)
    assert (a1 == a2).all()
    w = configs.gen_w(case)
    assert (tx.pack_ternary(w) == configs.gen_w_packed(case)).all()
    frac = np.bincount((w.ravel() + 1).astype(np.int64), minlength=3) / w.size
    assert abs(frac[0] - 0.3) < 0.01 and abs(frac[1] - 0.4) < 0.01 and abs(frac[2] - 0.3) < 0.01
    # element i depends only on i: a prefix of a larger array equals the smaller array
    big = np.empty(10_000_000, np.int8)
    lib.ternix_synth_act_uniform(big.ctypes.data_as(ctypes.c_void_p), big.size, 0, 2 * case.stream)
    assert (big[: a1.size] == a1.ravel()).all()


def test_gauss_distribution():
    a = configs.gen_a(configs.CASES["cfg3_m64_up"])
    assert abs(float(a.mean())) < 0.5 and 30.5 < float(a.std()) < 32.5
    assert a.min() >= -128 and a.max() <= 127


def test_device_bitpack_validation_without_launch():
    """Null device pointers are rejected before any HIP call; nothing to do for fewer than 4 weights."""
    lib = tx._load()
    for name in ("ternix_hip_pack_ternary_weights", "ternix_hip_unpack_ternary_weights",
                 "ternix_hip_interleave_weights_offline"):
        fn = getattr(lib, name)
        assert fn(None, None, 64, None) == 1, name
        assert fn(None, None, 3, None) == 0, name
