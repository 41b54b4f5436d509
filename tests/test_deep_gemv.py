"""The whole-K deep GEMV (skinny_deep.hip), automatic on tile-64 weights for short-K decode shapes
and forced here through the test hook on both layouts and for every built configuration, against
the CPU oracle (bit-exact), with K splits through the reduce launch and with the dequantising
epilogue (bit-equal to the default path's floats)."""
import numpy as np
import pytest

import ternixengine_amd as tx
from ternixengine_amd import hip_runtime as hr

CONFIGS = [(16, 16, 4), (16, 16, 8), (16, 8, 4), (16, 8, 8)]
SHAPES = [(1, 64, 64), (1, 2560, 2560), (3, 640, 1024), (4, 4096, 1088), (5, 1536, 512), (16, 2560, 6912),
          (13, 192, 4160), (1, 6912, 2560)]


@pytest.fixture
def lib():
    lib = tx._load()
    lib.ternix_hip_debug_reset()
    yield lib
    lib.ternix_hip_debug_reset()


def _inputs(m, k, n, seed):
    rng = np.random.default_rng(seed)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    return a, wp


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: "nw%d_nsw%d" % c[1:])
@pytest.mark.parametrize("splits", [1, 2, 3])
def test_deep_forced_row_major(lib, oracle, cfg, splits):
    for i, (m, k, n) in enumerate(SHAPES):
        a, wp = _inputs(m, k, n, 100 + i)
        assert lib.ternix_hip_debug_set(b"deep", *cfg, splits) == 0
        print(f"deep {cfg} splits {splits} M={m} K={k} N={n}", flush=True)
        da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n)
        dc.upload(np.full(m * n, -7, np.int32))
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
        hr.synchronize()
        assert (dc.download(np.int32, (m, n)) == oracle.mm("scalar_mt", a, wp, n)).all(), (m, k, n)


@pytest.mark.gpu
@pytest.mark.parametrize("forced", [None, (16, 16, 4, 1), (16, 8, 8, 2)])
def test_deep_tile64(lib, oracle, forced):
    # tile-64 contract: K % 128, N % 256; M <= 16 and K <= 4096 take the deep kernel automatically
    for i, (m, k, n) in enumerate([(1, 2560, 6912), (4, 4096, 11008), (16, 2560, 2560), (7, 128, 256),
                                   (1, 6912, 2560)]):
        a, wp = _inputs(m, k, n, 300 + i)
        if forced:
            assert lib.ternix_hip_debug_set(b"deep", *forced) == 0
        print(f"tile64 deep {forced} M={m} K={k} N={n}", flush=True)
        got = tx.ternary_matmul_tile64(a, tx.interleave_tile64(wp), n)
        assert (got == oracle.mm("scalar_mt", a, wp, n)).all(), (m, k, n)


@pytest.mark.gpu
def test_deep_dequant_matches_default(lib):
    m, k, n = 4, 2560, 6912
    a, wp = _inputs(m, k, n, 7)
    rs = np.linspace(0.01, 0.04, m).astype(np.float32)
    ref = tx.ternary_matmul_dequant(a, wp, rs, 0.37)
    for splits in (1, 2):
        assert lib.ternix_hip_debug_set(b"deep", 16, 16, 4, splits) == 0
        got = tx.ternary_matmul_dequant(a, wp, rs, 0.37)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), splits
