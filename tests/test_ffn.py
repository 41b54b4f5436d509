"""Feed-forward block on the GPU: RMSNorm and SwiGLU against the reference's own routines
(src/simd_math.cpp, compiled into oracle/_ref when the sources are present, and their plain-C
restatement in oracle/), the SwiGLU-fused up-projection, and the four-launch ternix_hip_ffn_forward.

Float tolerances: RMSNorm's sum of squares is a parallel tree on the GPU and a sequential sum in the
reference, so they agree to float rounding -- tested at 1e-5 relative (the reference holds its own
scalar and AVX2 versions to 1e-4, tests/test_simd_math.cpp:17-27).  exp differs between the GPU math
library and glibc by at most an ulp or two: SwiGLU outputs are held to 1e-6 relative.  Integer and
dequantisation steps stay bit-exact."""
import ctypes
import os
import sys

import numpy as np
import pytest

import ternixengine_amd as tx
from conftest import ROOT

F32 = np.float32
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libternix_ref.so")


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _ref():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (reference sources absent)")
    lib = ctypes.CDLL(REF_SO)
    for n in ("ref_rms_norm_scalar", "ref_rms_norm_avx2"):
        getattr(lib, n).argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_size_t, ctypes.c_float]
    lib.ref_swiglu.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    return lib


def o_rms(oracle, x, w, eps):
    x = np.ascontiguousarray(x, F32)
    out = np.empty_like(x)
    oracle.lib.oracle_rms_norm.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_size_t, ctypes.c_float]
    for r in range(x.shape[0]):
        oracle.lib.oracle_rms_norm(_p(out[r]), _p(x[r]), _p(w), x.shape[1], eps)
    return out


def o_swiglu(oracle, x):
    x = np.ascontiguousarray(x, F32).reshape(-1)
    out = np.empty(x.size // 2, F32)
    oracle.lib.oracle_swiglu(_p(out), _p(x), ctypes.c_size_t(x.size))
    return out


def o_quant(oracle, x):
    x = np.ascontiguousarray(x, F32)
    m, k = x.shape
    q, rs = np.empty((m, k), np.int8), np.empty(m, F32)
    oracle.lib.oracle_quantize_rows_absmax(_p(x), _p(q), _p(rs), ctypes.c_size_t(m), ctypes.c_size_t(k))
    return q, rs


def dequant_np(c, rs, ws):
    return c.astype(F32) * (rs[:, None].astype(F32) * F32(ws))


# ---------------------------------------------------------------- oracle pinning (CPU)

def test_oracle_rms_norm_known_value(oracle):
    x = np.array([[1, 2, 3, 4]], F32)  # reference tests/test_simd_math.cpp:7-15
    out = o_rms(oracle, x, np.ones(4, F32), 1e-5)
    rms = np.sqrt((1 + 4 + 9 + 16) / 4.0 + 1e-5)
    assert abs(out[0, 0] - 1 / rms) < 1e-4 and abs(out[0, 3] - 4 / rms) < 1e-4


def test_oracle_swiglu_known_value(oracle):
    out = o_swiglu(oracle, np.array([1.0, 2.0], F32))  # reference tests/test_simd_math.cpp:29-35
    assert abs(out[0] - 2.0 / (1.0 + np.exp(-1.0))) < 1e-6


@pytest.mark.parametrize("n", [1, 7, 8, 9, 64, 100, 4096])
def test_oracle_matches_compiled_reference(oracle, n):
    lib = _ref()
    rng = np.random.default_rng(7 + n)
    x, w = rng.normal(0, 2, n).astype(F32), rng.normal(0, 2, n).astype(F32)
    a, b = np.empty(n, F32), np.empty(n, F32)
    lib.ref_rms_norm_scalar(_p(a), _p(x), _p(w), n, 1e-5)
    lib.ref_rms_norm_avx2(_p(b), _p(x), _p(w), n, 1e-5)
    mine = o_rms(oracle, x[None], w, 1e-5)[0]
    # the reference build may contract the sum of squares into FMAs: equal to a few ulps
    np.testing.assert_allclose(mine, a, rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(mine, b, rtol=1e-4, atol=1e-30)
    s = rng.normal(0, 3, 2 * n + 1).astype(F32)
    r = np.empty(n, F32)
    lib.ref_swiglu(_p(r), _p(s), s.size)
    np.testing.assert_array_equal(o_swiglu(oracle, s), r)


# ---------------------------------------------------------------- GPU

gpu = pytest.mark.gpu


@gpu
@pytest.mark.parametrize("shape", [(1, 1), (1, 7), (3, 8), (2, 9), (5, 64), (4, 100), (2, 4096), (16, 2560)])
def test_gpu_rms_norm(oracle, shape):
    log(f"[rms_norm] {shape}")
    rng = np.random.default_rng(sum(shape))
    x = rng.normal(0, 2, shape).astype(F32)
    w = rng.normal(0, 2, shape[1]).astype(F32)
    np.testing.assert_allclose(tx.rms_norm(x, w, 1e-5), o_rms(oracle, x, w, 1e-5), rtol=1e-5, atol=1e-6)


@gpu
@pytest.mark.parametrize("size", [2, 3, 1000, 13824, 1 << 20])
def test_gpu_swiglu(oracle, size):
    log(f"[swiglu] {size}")
    x = np.random.default_rng(size).normal(0, 4, size).astype(F32)
    np.testing.assert_allclose(tx.swiglu(x), o_swiglu(oracle, x), rtol=1e-6, atol=1e-30)


def _dev(a):
    from ternixengine_amd import hip_runtime as hr
    return hr.DeviceBuffer.from_array(np.ascontiguousarray(a))


@gpu
@pytest.mark.parametrize("shape", [(1, 2560), (8, 1024), (64, 4096)])
def test_gpu_rms_norm_quantize(oracle, shape):
    from ternixengine_amd import hip_runtime as hr
    log(f"[rms_norm_quantize] {shape}")
    m, k = shape
    rng = np.random.default_rng(m * k)
    x, w = rng.normal(0, 2, shape).astype(F32), rng.normal(1, 0.2, k).astype(F32)
    dx, dw, dq, ds = _dev(x), _dev(w), hr.DeviceBuffer(m * k), hr.DeviceBuffer(4 * m)
    assert tx._load().ternix_hip_rms_norm_quantize(dq.value, ds.value, dx.value, dw.value, m, k, 1e-5, None) == 0
    hr.synchronize()
    q, rs = dq.download(np.int8, (m, k)), ds.download(F32, (m,))
    qo, rso = o_quant(oracle, o_rms(oracle, x, w, 1e-5))
    np.testing.assert_allclose(rs, rso, rtol=1e-5)
    diff = np.abs(q.astype(np.int32) - qo)
    assert diff.max() <= 1 and (diff > 0).mean() < 1e-3   # only values within rounding of a .5 tie move


def _ffn_weights(rng, h, f):
    t_gu = (rng.integers(0, 10, size=(h, 2 * f)) // 4 - 1).clip(-1, 1).astype(np.int8)
    t_d = (rng.integers(0, 10, size=(f, h)) // 4 - 1).clip(-1, 1).astype(np.int8)
    return t_gu, t_d


@gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (4, 4096, 1024), (48, 1024, 512), (16, 640, 130)])
def test_gpu_swiglu_matmul(oracle, shape):
    from ternixengine_amd import hip_runtime as hr
    m, k, f = shape
    log(f"[swiglu matmul] M={m} K={k} F={f}")
    rng = np.random.default_rng(m + k + f)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    t = (rng.integers(0, 10, size=(k, 2 * f)) // 4 - 1).clip(-1, 1).astype(np.int8)
    wp = tx.pack_ternary(t)
    rs = rng.uniform(1e-4, 1e-3, size=m).astype(F32)
    da, db, drs = _dev(a), _dev(wp), _dev(rs)
    dh, dsc = hr.DeviceBuffer(4 * m * f), hr.DeviceBuffer(8 * m * f)
    st = tx._load().ternix_hip_mul_mat_ternary_swiglu(da.value, db.value, dh.value, m, k, 2 * f, drs.value, 0.5,
                                                      dsc.value, None)
    assert st == 0, tx.ternix_error(st)
    hr.synchronize()
    h = dh.download(F32, (m, f))
    y = dequant_np(oracle.mm("scalar", a, wp, 2 * f), rs, 0.5)   # bit-exact dequantised product
    want = o_swiglu(oracle, y).reshape(m, f)
    np.testing.assert_allclose(h, want, rtol=1e-6, atol=1e-30)


@gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (4, 1024, 2048), (64, 512, 1024)])
def test_gpu_ffn_forward(oracle, shape):
    """The four-launch block equals its pieces run one by one through the public entry points (bit
    for bit), and approximates the unquantised float64 block."""
    from ternixengine_amd import hip_runtime as hr
    m, hd, f = shape
    log(f"[ffn] M={m} H={hd} F={f}")
    rng = np.random.default_rng(m + hd + f)
    x = rng.normal(0, 1, (m, hd)).astype(F32)
    g = rng.normal(1, 0.1, hd).astype(F32)
    t_gu, t_d = _ffn_weights(rng, hd, f)
    wgu, wd = tx.pack_ternary(t_gu), tx.pack_ternary(t_d)
    ws_gu, ws_d = 0.02, 0.03
    y = tx.ffn_forward(x, g, 1e-5, wgu, ws_gu, wd, ws_d)

    lib = tx._load()
    dx, dg, dgu, dd = _dev(x), _dev(g), _dev(wgu), _dev(wd)
    dq1, drs1 = hr.DeviceBuffer(m * hd), hr.DeviceBuffer(4 * m)
    dh, dsc = hr.DeviceBuffer(4 * m * f), hr.DeviceBuffer(8 * m * f)
    dq2, drs2, dy = hr.DeviceBuffer(m * f), hr.DeviceBuffer(4 * m), hr.DeviceBuffer(4 * m * hd)
    assert lib.ternix_hip_rms_norm_quantize(dq1.value, drs1.value, dx.value, dg.value, m, hd, 1e-5, None) == 0
    assert lib.ternix_hip_mul_mat_ternary_swiglu(dq1.value, dgu.value, dh.value, m, hd, 2 * f, drs1.value, ws_gu,
                                                 dsc.value, None) == 0
    assert lib.ternix_hip_quantize_activations(dh.value, dq2.value, drs2.value, m, f, None) == 0
    assert lib.ternix_hip_mul_mat_ternary_dequant(dq2.value, dd.value, dy.value, m, f, hd, drs2.value, ws_d,
                                                  None) == 0
    hr.synchronize()
    np.testing.assert_array_equal(y, dy.download(F32, (m, hd)))

    xn = o_rms(oracle, x, g, 1e-5).astype(np.float64)
    u = xn @ (t_gu.astype(np.float64) * ws_gu)
    hh = (u[:, 0::2] / (1 + np.exp(-u[:, 0::2]))) * u[:, 1::2]
    ref = hh @ (t_d.astype(np.float64) * ws_d)
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 0.03, rel   # int8 activation quantisation twice: ~1% relative error


@gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (4, 2560, 6912), (3, 1024, 2304), (16, 1024, 2816),
                                   (24, 512, 1024)])
def test_gpu_ffn_forward_tile64(shape):
    """The block on tile-64 weights equals the block on the contract layout, bit for bit (up to 4 rows
    the two whole-line GEMV launches on the tile-64 blocks, fused RMSNorm + quantisation in the gate/up
    GEMV up to 16 rows, the separate launches above)."""
    m, hd, f = shape
    log(f"[ffn tile-64] M={m} H={hd} F={f}")
    rng = np.random.default_rng(7 * m + hd + f)
    x = rng.normal(0, 1, (m, hd)).astype(F32)
    g = rng.normal(1, 0.1, hd).astype(F32)
    t_gu, t_d = _ffn_weights(rng, hd, f)
    wgu, wd = tx.pack_ternary(t_gu), tx.pack_ternary(t_d)
    y = tx.ffn_forward(x, g, 1e-5, wgu, 0.02, wd, 0.03)
    yt = tx.ffn_forward_tile64(x, g, 1e-5, wgu, 0.02, wd, 0.03)
    np.testing.assert_array_equal(yt, y)


def test_ffn_validation():
    lib = tx._load()
    assert lib.ternix_hip_ffn_workspace_size(1, 2560, 6912) > 0
    # H % 4 and F % 2 are checked before any pointer is used
    assert lib.ternix_hip_ffn_forward(None, None, None, 1e-5, None, 1.0, None, 1.0, 1, 6, 4, None, 0, None) == 1
    # tile-64: H % 256 and F % 128 are checked before any pointer is used
    assert lib.ternix_hip_ffn_forward_tile64(None, None, None, 1e-5, None, 1.0, None, 1.0, 1, 2560, 64, None, 0,
                                             None) == 1
    assert lib.ternix_hip_ffn_forward_tile64(None, None, None, 1e-5, None, 1.0, None, 1.0, 1, 2500, 6912, None, 0,
                                             None) == 1
    assert lib.ternix_hip_ffn_forward(None, None, None, 1e-5, None, 1.0, None, 1.0, 1, 8, 3, None, 0, None) == 1
    assert lib.ternix_hip_ffn_forward(None, None, None, 1e-5, None, 1.0, None, 1.0, 1, 8, 4, None, 0, None) == 1
    assert lib.ternix_hip_swiglu(None, None, 1, None) == 0
    assert lib.ternix_hip_rms_norm(None, None, None, 1, 4, 1e-5, None) == 1


@gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (4, 1024, 2048)])
def test_gpu_ffn_graph_replays_match_eager(shape):
    """ffn_forward recorded into a hipGraph on a fresh stream (its split-K matmuls are first used
    inside the capture, so they take the zero-fill + atomic path through the caller's scratch) and
    replayed several times, with eager work on another stream in between: every replay equals the
    eager result (partial-sum path) bit for bit."""
    from ternixengine_amd import hip_runtime as hr
    m, hd, f = shape
    log(f"[ffn graph] M={m} H={hd} F={f}")
    rng = np.random.default_rng(17 + m)
    x = rng.normal(0, 1, (m, hd)).astype(F32)
    g = rng.normal(1, 0.1, hd).astype(F32)
    t_gu, t_d = _ffn_weights(rng, hd, f)
    wgu, wd = tx.pack_ternary(t_gu), tx.pack_ternary(t_d)
    eager = tx.ffn_forward(x, g, 1e-5, wgu, 0.02, wd, 0.03)
    lib = tx._load()
    nws = lib.ternix_hip_ffn_workspace_size(m, hd, f)
    dx, dg, dgu, dd = _dev(x), _dev(g), _dev(wgu), _dev(wd)
    dy, dws = hr.DeviceBuffer(4 * m * hd), hr.DeviceBuffer(nws)
    s = hr.Stream()
    graph = hr.Graph(s, lambda: lib.ternix_hip_ffn_forward(dy.value, dx.value, dg.value, 1e-5, dgu.value, 0.02,
                                                           dd.value, 0.03, m, hd, f, dws.value, nws, s.handle))
    for rep in range(4):
        dy.upload(np.full(m * hd, np.nan, F32))
        graph.launch()
        s.synchronize()
        np.testing.assert_array_equal(dy.download(F32, (m, hd)), eager, err_msg=f"replay {rep}")
        tx.ffn_forward(x, g, 1e-5, wgu, 0.02, wd, 0.03)  # eager work between replays
