"""Quantised layer boundary: absmax activation quantisation, fused dequantising matmul, absmean weight
quantisation (include/ternix/ternix_hip.h).  The reference has no implementation of these (it stubs
them: scripts/quantize.py:5, README.md:203), so the oracle restates the documented BitNet b1.58
formulas and is pinned here by closed forms and by an independent numpy float32 evaluation; the GPU
is then held to bit equality with the oracle (every step is IEEE fp32 with one rounding each)."""
import ctypes
import sys

import numpy as np
import pytest

import ternixengine_amd as tx

F32 = np.float32


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def oracle_quant(oracle, x):
    x = np.ascontiguousarray(x, dtype=F32)
    m, k = x.shape
    q, rs = np.empty((m, k), np.int8), np.empty(m, F32)
    oracle.lib.oracle_quantize_rows_absmax(_p(x), _p(q), _p(rs), ctypes.c_size_t(m), ctypes.c_size_t(k))
    return q, rs


def oracle_dequant(oracle, c, rs, ws):
    c = np.ascontiguousarray(c, dtype=np.int32)
    rs = np.ascontiguousarray(rs, dtype=F32)
    y = np.empty(c.shape, F32)
    oracle.lib.oracle_dequant.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_float, ctypes.c_size_t, ctypes.c_size_t]
    oracle.lib.oracle_dequant(_p(c), _p(y), _p(rs), ws, c.shape[0], c.shape[1])
    return y


def oracle_wquant(oracle, w):
    w = np.ascontiguousarray(w, dtype=F32)
    q = np.empty(w.shape, np.int8)
    oracle.lib.oracle_quantize_weights_absmean.restype = ctypes.c_float
    g = oracle.lib.oracle_quantize_weights_absmean(_p(q), _p(w), ctypes.c_size_t(w.size))
    return q, float(g)


def numpy_quant(x):
    """Independent float32 evaluation of the same formula (numpy float32 ops are IEEE)."""
    x = x.astype(F32)
    a = np.maximum(np.abs(x).max(axis=1), F32(1e-5)).astype(F32)
    s = (F32(127.0) / a).astype(F32)
    q = np.clip(np.rint((x * s[:, None]).astype(F32)), -128, 127).astype(np.int8)
    return q, (a / F32(127.0)).astype(F32)


# ---------------------------------------------------------------- oracle pinning (CPU)

def test_quant_closed_forms(oracle):
    x = np.zeros((4, 8), F32)
    x[1] = [127, -127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]   # absmax 127: scale exactly 1, ties to even
    x[2] = 3.0                                           # constant row -> all 127
    x[3] = [-8, 4, 2, 1, 0, -1, -2, -4]                  # absmax 8: scale 127/8 (exact), q = 127*x/8
    q, rs = oracle_quant(oracle, x)
    assert (q[0] == 0).all() and rs[0] == F32(1e-5) / F32(127)
    assert q[1].tolist() == [127, -127, 0, 2, 2, 0, -2, -2]
    assert rs[1] == F32(1.0)
    assert (q[2] == 127).all()
    assert q[3].tolist() == [-127, 64, 32, 16, 0, -16, -32, -64]   # rint(63.5) = 64, rint(15.875) = 16
    perm = np.array([2, 0, 3, 1])
    q2, rs2 = oracle_quant(oracle, x[perm])
    np.testing.assert_array_equal(q2, q[perm])
    np.testing.assert_array_equal(rs2, rs[perm])


def test_quant_matches_numpy_float32(oracle):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((37, 1000)) * rng.uniform(0.01, 100, size=(37, 1))).astype(F32)
    q, rs = oracle_quant(oracle, x)
    qn, rsn = numpy_quant(x)
    np.testing.assert_array_equal(q, qn)
    np.testing.assert_array_equal(rs, rsn)
    # and the quantisation error is at most half a step
    err = np.abs(q.astype(np.float64) * rs[:, None] - x)
    assert (err <= 0.5 * rs[:, None] * (1 + 1e-6)).all()


def test_dequant_closed_forms(oracle):
    c = np.array([[0, 1, -1, 1 << 24], [123456, -7, 2**31 - 1, -2**31]], np.int32)
    rs = np.array([0.25, 2.0], F32)
    y = oracle_dequant(oracle, c, rs, 0.5)
    # power-of-two scales: exact products of the fp32-rounded integers
    np.testing.assert_array_equal(y, c.astype(F32) * (rs[:, None] * F32(0.5)))
    assert y[0, 3] == 2 ** 24 / 8 and y[1, 3] == -(2 ** 31)


def test_weight_quant_recovers_scaled_ternary(oracle):
    rng = np.random.default_rng(5)
    t = rng.choice(np.array([-1, 0, 1], np.int8), size=(64, 128), p=[0.4, 0.2, 0.4])
    w = (t * F32(0.375)).astype(F32)                   # mean|W| = 0.375 * 0.8 = 0.3 -> W/gamma = +-1.25
    q, g = oracle_wquant(oracle, w)
    np.testing.assert_array_equal(q, t)
    assert abs(g - 0.375 * (t != 0).mean()) < 1e-7
    packed, g_lib = tx.quantize_weights_absmean(w)    # the library's host routine agrees bit for bit
    assert g_lib == g
    np.testing.assert_array_equal(tx.unpack_ternary(packed), q)
    qz, gz = oracle_wquant(oracle, np.zeros((4, 8), F32))
    assert (qz == 0).all() and gz == F32(1e-5)


def test_weight_quant_random_matches_library(oracle):
    rng = np.random.default_rng(9)
    w = (rng.integers(-4096, 4097, size=(96, 64)) / F32(1024)).astype(F32)  # exact double sums
    q, g = oracle_wquant(oracle, w)
    packed, g_lib = tx.quantize_weights_absmean(w)
    assert g_lib == g and g == F32(np.abs(w.astype(np.float64)).mean())
    np.testing.assert_array_equal(tx.unpack_ternary(packed), q)
    np.testing.assert_array_equal(q, np.clip(np.rint(w / F32(g)), -1, 1).astype(np.int8))


# ---------------------------------------------------------------- GPU parity

gpu = pytest.mark.gpu


@gpu
@pytest.mark.parametrize("shape", [(1, 2560), (4, 4096), (17, 1000), (64, 11008), (3, 1), (5, 33), (2048, 64)])
def test_gpu_quantize_matches_oracle(oracle, shape):
    log(f"[quantize] shape={shape}")
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(shape) * rng.uniform(0.01, 50, size=(shape[0], 1))).astype(F32)
    if shape[0] > 2:
        x[0, :] = 0.0  # an all-zero row
    q, rs = tx.quantize_activations(x)
    qo, rso = oracle_quant(oracle, x)
    np.testing.assert_array_equal(q, qo)
    np.testing.assert_array_equal(rs, rso)


def _mm_oracle(oracle, a, wp, n):
    return oracle.mm("scalar", a, wp, n)


@gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (1, 6912, 2560), (4, 4096, 1024), (16, 1024, 512),
                                   (32, 640, 256), (64, 1024, 512), (129, 1000, 260), (2048, 512, 1024),
                                   (1, 1000, 3076), (17, 4093, 1028)])
def test_gpu_dequant_matmul_matches_oracle(oracle, shape):
    m, k, n = shape
    log(f"[dequant matmul] M={m} K={k} N={n}")
    rng = np.random.default_rng(m + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    w = (rng.integers(0, 10, size=(k, n)) // 4 - 1).clip(-1, 1).astype(np.int8)
    wp = tx.pack_ternary(w)
    rs = rng.uniform(1e-3, 1.0, size=m).astype(F32)
    ws = 0.4375
    y = tx.ternary_matmul_dequant(a, wp, rs, ws)
    yo = oracle_dequant(oracle, _mm_oracle(oracle, a, wp, n), rs, ws)
    np.testing.assert_array_equal(y, yo)


@gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (1, 6912, 2560), (4, 4096, 1024), (24, 2048, 1024),
                                   (64, 1024, 512), (200, 1024, 512)])
def test_gpu_tile64_dequant_matches_oracle(oracle, shape):
    """The dequantising matmul on tile-64 weights: the same float outputs, bit for bit."""
    m, k, n = shape
    log(f"[tile-64 dequant matmul] M={m} K={k} N={n}")
    rng = np.random.default_rng(m * 3 + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    w = (rng.integers(0, 10, size=(k, n)) // 4 - 1).clip(-1, 1).astype(np.int8)
    wp = tx.pack_ternary(w)
    rs = rng.uniform(1e-3, 1.0, size=m).astype(F32)
    ws = 0.4375
    y = tx.ternary_matmul_tile64_dequant(a, tx.interleave_tile64(wp), n, rs, ws)
    yo = oracle_dequant(oracle, _mm_oracle(oracle, a, wp, n), rs, ws)
    np.testing.assert_array_equal(y, yo)


@gpu
def test_gpu_dequant_long_k_chunks_and_misaligned(oracle):
    """K beyond one accumulator (int32 chunks kept in Y, converted in place) and a Y that is not
    16-byte aligned (scalar stores)."""
    from ternixengine_amd import hip_runtime as hr
    for (m, k, n, off) in ((33, (1 << 17) + 64, 64, 0), (2, (1 << 17) + 64, 64, 0), (40, 256, 128, 4),
                           (3, 512, 128, 4)):
        log(f"[dequant] M={m} K={k} N={n} y_offset={off}")
        rng = np.random.default_rng(k + off)
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        w = (rng.integers(0, 3, size=(k, n)) - 1).astype(np.int8)
        wp = tx.pack_ternary(w)
        rs = rng.uniform(1e-3, 1.0, size=m).astype(F32)
        da, db, drs = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer.from_array(rs)
        dy = hr.DeviceBuffer(4 * m * n + off + 16)
        st = tx._load().ternix_hip_mul_mat_ternary_dequant(da.value, db.value, dy.value + off, m, k, n, drs.value,
                                                          0.75, None)
        assert st == 0, tx.ternix_error(st)
        hr.synchronize()
        y = dy.download(np.uint8, (4 * m * n + off + 16,))[off:off + 4 * m * n].view(F32).reshape(m, n)
        np.testing.assert_array_equal(y, oracle_dequant(oracle, _mm_oracle(oracle, a, wp, n), rs, 0.75))


@gpu
def test_gpu_layer_boundary_end_to_end(oracle):
    """fp32 activations and weights -> quantise both -> fused dequantising matmul, against the oracle
    bit for bit and against the fp32 product within the quantisation error."""
    rng = np.random.default_rng(11)
    m, k, n = 8, 2048, 1024
    x = rng.standard_normal((m, k)).astype(F32)
    wf = (rng.standard_normal((k, n)) * 0.02).astype(F32)
    wp, ws = tx.quantize_weights_absmean(wf)
    q, rs = tx.quantize_activations(x)
    y = tx.ternary_matmul_dequant(q, wp, rs, ws)
    qo, rso = oracle_quant(oracle, x)
    yo = oracle_dequant(oracle, _mm_oracle(oracle, qo, wp, n), rso, ws)
    np.testing.assert_array_equal(y, yo)
    # the product of the dequantised operands, in float64, is what y approximates to fp32 rounding
    ref = (q.astype(np.float64) * rs[:, None].astype(np.float64)) @ (tx.unpack_ternary(wp).astype(np.float64) * ws)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
