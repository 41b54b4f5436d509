"""ternix_hip_mul_mat_ternary_noalloc (fixed device scratch, no allocation) against
ternix_hip_mul_mat_ternary on the same inputs: bit-identical outputs, two calls in a row with the
second on a smaller input, no device allocation by the library during the calls, and the size
limit rejected with hipErrorOutOfMemory before any work."""
import numpy as np
import pytest

import ternixengine_amd as tx
from ternixengine_amd import hip_runtime as hr

# Each pair: a larger call, then a smaller one (the second reuses scratch the first left behind).
PAIRS = [
    ((16, 11008, 4096), (4, 4096, 1024)),     # GEMV split partials, then a smaller split
    ((1, 8192, 28672), (1, 2560, 6912)),      # DMA-staged GEMV + reduce, then the wave GEMV
    ((64, 11008, 4096), (40, 6144, 2048)),    # GEMM split-K, then a smaller split
    ((129, 8191, 2052), (17, 4093, 1028)),    # ragged: padded copies of W and A, then smaller ones
    ((256, 4096, 4096), (1, 1000, 3076)),     # GEMM without scratch, then ragged GEMV
    ((256, 16384, 4096), (128, 11008, 4096)),  # split-K 64-row tiles (16 MiB of partials), then 8 splits
]


def _inputs(rng, m, k, n):
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    return hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp)


@pytest.mark.gpu
@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: "%dx%dx%d-then-%dx%dx%d" % (p[0] + p[1]))
def test_noalloc_matches_auto(pair):
    lib = tx._load()
    rng = np.random.default_rng(sum(pair[0]) + sum(pair[1]))
    for m, k, n in pair:
        print(f"noalloc M={m} K={k} N={n}", flush=True)
        assert lib.ternix_hip_mul_mat_ternary_workspace_size(m, k, n) <= lib.ternix_hip_noalloc_scratch_bytes()
        da, db = _inputs(rng, m, k, n)
        ref_c, got_c = hr.DeviceBuffer(4 * m * n), hr.DeviceBuffer(4 * m * n)
        got_c.upload(np.full(m * n, -7, np.int32))
        assert lib.ternix_hip_mul_mat_ternary(da.value, db.value, ref_c.value, m, k, n, None) == 0
        hr.synchronize()
        before = lib.ternix_hip_debug_alloc_count()
        assert lib.ternix_hip_mul_mat_ternary_noalloc(da.value, db.value, got_c.value, m, k, n, None) == 0
        hr.synchronize()
        assert lib.ternix_hip_debug_alloc_count() == before
        assert (got_c.download(np.int32, (m, n)) == ref_c.download(np.int32, (m, n))).all(), (m, k, n)


@pytest.mark.gpu
def test_noalloc_rejects_oversize_and_bad_shape():
    lib = tx._load()
    # a GEMV with a long K split over many workgroups: [splits][M][N] int32 partials of 68 MiB
    m, k, n = 16, 65536, 32768
    need = lib.ternix_hip_mul_mat_ternary_workspace_size(m, k, n)
    assert need > lib.ternix_hip_noalloc_scratch_bytes(), need
    assert lib.ternix_hip_mul_mat_ternary_noalloc(1 << 20, 1 << 24, 1 << 20, m, k, n, None) == 2
    assert lib.ternix_hip_mul_mat_ternary_noalloc(1 << 20, 1 << 24, 1 << 20, 1, 64, 6, None) == 1
