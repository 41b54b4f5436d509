"""The kernels the automatic dispatch only falls back to (register-staged skinny kernels, generic
kernels for ragged shapes, 256-column GEMM tiles for small M, the reduce launch instead of in-launch
split sums, the generic GEMM, the self-zeroing wave kernel that the whole-line GEMV replaces for most
M <= 4 shapes) stay bit-exact.  Each switch set is applied in-process through the
library's explicit test hook, ternix_hip_debug_set (the library never reads the environment)."""
import numpy as np
import pytest

import ternixengine_amd as tx
from ternixengine_amd import hip_runtime as hr

SHAPES = [(1, 2560, 2560), (1, 6912, 2560), (4, 4096, 1024), (16, 2048, 4096), (16, 8192, 1024), (24, 4096, 512),
          (32, 2560, 1024), (48, 1024, 2048), (64, 4096, 1024), (129, 1001, 516), (1, 1000, 3076), (17, 4093, 1028),
          (256, 2048, 1024), (320, 1024, 2048), (96, 8192, 1024), (256, 6144, 1024)]

SWITCHES = [
    {"skinny_wave": 0},                                    # DMA-staged GEMVs
    {"wave_sw": 16},                                       # 16-byte wave strips
    {"skinny_wave": 0, "skinny_dma": 0},                   # short / fast kernels
    {"skinny_wave": 0, "skinny_dma": 0, "skinny_short": 0},  # fast kernel only
    {"ragged_pad": 0},                                     # generic ragged kernels
    {"gemm_narrow": 0},                                    # 256-column small-M GEMM
    {"wave_last": 0},                                      # reduce launch instead of in-launch sums
    {"gemm_generic": 1},                                   # register-staged generic GEMM
    {"sk_order": 1},                                       # release/acquire form of the in-launch sums
    {"m1_atomic": 0},                                      # M = 1 without the zero-fill + atomic plan
    {"m1_atomic": 0, "sk_order": 1},                       # ... and its in-launch sums in release/acquire form
    {"self_zero": 0},                                      # M = 1 atomic plan with the fill launch
    {"gemm_bm": 128},                                      # 128-row GEMM tiles of eight waves
    {"gemm_bm": 256},                                      # 256-row GEMM tiles
    {"gemm_bm": 64},                                       # 64-row GEMM tiles, split or not
    {"gemm_narrow": 1},                                    # 64 x 64 GEMM tiles at any M and split
    {"gemm_splits": 3},                                    # an odd GEMM split count
    {"nt": (1, 1)},                                        # non-temporal weight loads in both GEMV kernels
    {"skinny_wave": 0, "nt": (1, 1)},                      # ... in the DMA-staged GEMVs on every shape
    {"skinny_wave": 0, "skinny_dma": (3, 12)},             # DMA-staged GEMVs with a forced split count
    {"wave_ticket": 1},                                    # split ticket waited in the first k-step everywhere
    {"wave_ticket": 0},                                    # ... and right after the prologue everywhere
    {"wave_sw": (-1, -1, 0)},                              # no column waves in the M <= 4 atomic plan
    {"wave_sw": (-1, -1, 1)},                              # column waves wherever the plan allows them
    {"line": (2, 4)},                                      # whole-line GEMV, 2 k-steps, 4 data waves, M <= 4
    {"line": (4, 8)},                                      # whole-line GEMV, 4 k-steps, 8 data waves
]


@pytest.fixture
def switches(request):
    lib = tx._load()
    lib.ternix_hip_debug_reset()
    if "line" not in request.param:  # the switched kernels, not the whole-line GEMV that precedes them
        assert lib.ternix_hip_debug_set(b"line", 0, -1, -1, -1) == 0
    for k, v in request.param.items():
        v = tuple(v) if isinstance(v, tuple) else (v,)
        v = v + (-1,) * (4 - len(v))
        assert lib.ternix_hip_debug_set(k.encode(), *v) == 0, k
    yield request.param
    lib.ternix_hip_debug_reset()


def test_debug_set_rejects_unknown_key():
    lib = tx._load()
    assert lib.ternix_hip_debug_set(b"no_such_switch", 1, -1, -1, -1) == 1
    assert lib.ternix_hip_debug_set(None, 1, -1, -1, -1) == 1


@pytest.mark.gpu
@pytest.mark.parametrize("switches", SWITCHES, ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()),
                         indirect=True)
def test_fallback_kernels_bit_exact(switches, oracle):
    rng = np.random.default_rng(5)
    for m, k, n in SHAPES:
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n)
        dc.upload(np.full(m * n, -7, np.int32))
        print(f"M={m} K={k} N={n} {switches}", flush=True)
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
        hr.synchronize()
        assert (dc.download(np.int32, (m, n)) == oracle.mm("scalar_mt", a, wp, n)).all(), (m, k, n)
