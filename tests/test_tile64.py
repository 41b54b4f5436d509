"""The opt-in tile-64 weight layout: conversion (host and device) and the matmul that reads it.

The layout is a permutation of the packed K x N/4 bytes (1 KB blocks of 64 k-rows x 16 bytes, block
(strip c, k-step s) at (c * K/64 + s) * 1024, row r of the step at 16-byte position
r ^ (8 * ((r / 16) % 2))).  The host conversion is pinned here against a numpy reshape/transpose
statement of that permutation; the device conversion must equal the host one byte for byte; the
matmul on converted weights must equal the CPU oracle on the original packed weights (oracle/,
a restatement of reference src/mul_mat_ternary.cpp) and the committed digests of the reference's own
outputs, bit for bit.
"""
import ctypes
import hashlib
import sys

import numpy as np
import pytest

import ternixengine_amd as tx
from ternixengine_amd import configs

GARBAGE = np.int32(-0x2A2A2A2B)


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def numpy_tile64(p):
    """Independent statement of the layout: (K, NB) -> blocks[strip][kstep][pos] of 16 bytes."""
    k, nb = p.shape
    blocks = p.reshape(k // 64, 64, nb // 16, 16).transpose(2, 0, 1, 3)  # strip, kstep, row, byte
    r = np.arange(64)
    pos = r ^ (8 * ((r // 16) % 2))
    out = np.empty_like(blocks)
    out[:, :, pos, :] = blocks
    return out.reshape(-1)


# ---- CPU ----

@pytest.mark.parametrize("k,nb", [(64, 16), (128, 32), (192, 48), (2560, 640)])
def test_host_conversion_matches_numpy_statement(k, nb):
    rng = np.random.default_rng(k + nb)
    p = rng.integers(0, 256, size=(k, nb), dtype=np.uint8)
    got = tx.interleave_tile64(p)
    np.testing.assert_array_equal(got, numpy_tile64(p))
    # a permutation: same multiset of 16-byte rows
    assert sorted(map(bytes, got.reshape(-1, 16))) == sorted(map(bytes, p.reshape(-1, 16)))


def test_host_conversion_known_positions():
    """Row r of k-step s of strip c lands at block (c, s), position r ^ 8 for r in 16..31, 48..63."""
    k, nb = 128, 32
    p = np.zeros((k, nb), np.uint8)
    p[17, 16:32] = 7     # strip 1, step 0, row 17 -> position 25
    p[64 + 3, 0:16] = 9  # strip 0, step 1, row 3 -> position 3
    got = tx.interleave_tile64(p).reshape(-1, 16)
    assert (got[(1 * 2 + 0) * 64 + 25] == 7).all()
    assert (got[(0 * 2 + 1) * 64 + 3] == 9).all()
    assert int(got.astype(np.int64).sum()) == 7 * 16 + 9 * 16


def test_host_conversion_validation():
    lib = tx._load()
    buf = np.zeros(4096, np.uint8)
    vp = buf.ctypes.data_as(ctypes.c_void_p)
    out = np.zeros(4096, np.uint8)
    op = out.ctypes.data_as(ctypes.c_void_p)
    assert lib.ternix_interleave_weights_tile64(op, vp, 64, 64) == 0
    assert lib.ternix_interleave_weights_tile64(op, vp, 32, 64) == 1    # K % 64
    assert lib.ternix_interleave_weights_tile64(op, vp, 64, 32) == 1    # (N/4) % 16
    assert lib.ternix_interleave_weights_tile64(op, vp, 64, 66) == 1    # N % 4
    assert lib.ternix_interleave_weights_tile64(vp, vp, 64, 64) == 1    # in place
    assert lib.ternix_interleave_weights_tile64(None, None, 0, 64) == 0  # nothing to do
    with pytest.raises(ValueError):
        tx.interleave_tile64(np.zeros((96, 16), np.uint8))


def test_device_entry_points_validate_before_launch():
    """Rejected shapes, null and misaligned pointers return hipErrorInvalidValue (1) before any HIP
    call (the addresses below are never dereferenced); empty problems return 0."""
    lib = tx._load()
    conv = lib.ternix_hip_interleave_weights_tile64
    assert conv(None, None, 0, 256, None) == 0
    assert conv(None, None, 64, 256, None) == 1
    assert conv(0x1000, 0x2000, 96, 256, None) == 1
    assert conv(0x1000, 0x2000, 64, 200, None) == 1
    assert conv(0x1000, 0x1000, 64, 256, None) == 1
    mm = lib.ternix_hip_mul_mat_ternary_tile64
    assert mm(0x1000, 0x2000, 0x3000, 0, 128, 256, None) == 0      # M == 0
    assert mm(0x1000, 0x2000, 0x3000, 1, 64, 256, None) == 1       # K % 128
    assert mm(0x1000, 0x2000, 0x3000, 1, 128, 128, None) == 1      # N % 256
    assert mm(0x1001, 0x2000, 0x3000, 1, 128, 256, None) == 1      # A misaligned
    assert mm(0x1000, 0x2008, 0x3000, 1, 128, 256, None) == 1      # W misaligned
    assert mm(0x1000, 0x2000, 0x3002, 1, 128, 256, None) == 1      # C misaligned
    assert mm(None, 0x2000, 0x3000, 1, 128, 256, None) == 1
    assert mm(0x1000, 0x2000, 0x3000, -1, 128, 256, None) == 1
    dq = lib.ternix_hip_mul_mat_ternary_tile64_dequant
    assert dq(0x1000, 0x2000, 0x3000, 0, 128, 256, 0x4000, 1.0, None) == 0      # M == 0
    assert dq(0x1000, 0x2000, 0x3000, 1, 64, 256, 0x4000, 1.0, None) == 1      # K % 128
    assert dq(0x1000, 0x2000, 0x3000, 1, 128, 200, 0x4000, 1.0, None) == 1     # N % 256 (and N % 4)
    assert dq(0x1000, 0x2000, 0x3000, 1, 128, 256, None, 1.0, None) == 1       # row scales


# ---- GPU ----

def _hr():
    from ternixengine_amd import hip_runtime as hr
    if hr.device_count() < 1:
        pytest.skip("no HIP device")
    return hr


def device_convert(hr, wp):
    k, nb = wp.shape
    din = hr.DeviceBuffer.from_array(np.ascontiguousarray(wp))
    dout = hr.DeviceBuffer(wp.nbytes + 64)
    dout.upload(np.full(wp.nbytes + 64, 0xA5, np.uint8))
    st = tx.interleave_tile64_device(dout.value, din.value, k, nb * 4)
    assert st == 0, tx.ternix_error(st)
    hr.synchronize()
    got = dout.download(np.uint8, (wp.nbytes + 64,))
    assert (got[wp.nbytes:] == 0xA5).all()  # nothing written past the matrix
    return dout, got[:wp.nbytes]


def run_tile64(hr, a, dwt, n):
    a = np.ascontiguousarray(a, np.int8)
    m, k = a.shape
    da = hr.DeviceBuffer.from_array(a)
    dc = hr.DeviceBuffer(4 * m * n)
    dc.upload(np.full(m * n, GARBAGE, np.int32))
    st = tx.mul_mat_ternary(da.value, dwt.value, dc.value, m, k, n, path="tile64")
    assert st == 0, tx.ternix_error(st)
    hr.synchronize()
    return dc.download(np.int32, (m, n))


@pytest.mark.gpu
@pytest.mark.parametrize("k,n", [(64, 64), (128, 256), (2560, 6912), (6912, 2560)])
def test_device_conversion_equals_host(k, n):
    hr = _hr()
    log(f"[tile64 convert] K={k} N={n}")
    rng = np.random.default_rng(k * 7 + n)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    _, got = device_convert(hr, wp)
    np.testing.assert_array_equal(got, tx.interleave_tile64(wp))


SHAPES = [(m, k, n) for m in (1, 2, 3, 4, 5, 8, 13, 16, 17, 31, 32, 33, 64, 65, 128, 200)
          for k, n in ((128, 256), (2560, 2560), (4224, 768), (6912, 1280))]


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_tile64_matches_oracle(oracle, m, k, n):
    """Every planner branch: the wave kernel with K splits summed inside the launch and with the
    reduce launch, low-M and 16-row groups, and the GEMMs (M > 32) with and without split-K."""
    hr = _hr()
    log(f"[tile64 matmul] M={m} K={k} N={n}")
    rng = np.random.default_rng(m * 1000 + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int16).astype(np.int8)
    w = rng.integers(-1, 2, size=(k, n), dtype=np.int8)
    wp = oracle.pack(w)
    dwt, _ = device_convert(hr, wp)
    got = run_tile64(hr, a, dwt, n)
    np.testing.assert_array_equal(got, oracle.mm("scalar_mt", a, wp, n))


@pytest.mark.gpu
def test_matmul_tile64_extremes(oracle):
    """Worst-case magnitude (A = -128, W = -1) and W = 0 at a long K."""
    hr = _hr()
    log("[tile64 matmul] extremes")
    m, k, n = 3, 16384, 512
    a = np.full((m, k), -128, np.int8)
    wp = oracle.pack(np.full((k, n), -1, np.int8))
    dwt, _ = device_convert(hr, wp)
    assert (run_tile64(hr, a, dwt, n) == 128 * k).all()
    dz, _ = device_convert(hr, np.zeros((k, n // 4), np.uint8))
    assert (run_tile64(hr, a, dz, n) == 0).all()
    del dwt, dz


TILE64_CASES = ["cfg1", "cfg2_up", "cfg2_down", "cfg3_m4_up", "cfg3_m4_down", "cfg3_m16_up", "cfg3_m16_down",
                "cfg3_m64_up", "cfg3_m64_down", "cfg5_big_m1", "cfg4_4096x4096", "cfg4_14336x4096", "cfg5_worst"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", TILE64_CASES)
def test_configs_tile64_digest(digests, name):
    """Benchmark configurations on converted weights: the SHA-256 of C equals the digest of the
    reference's own output on the original packed weights."""
    hr = _hr()
    case = configs.CASES[name]
    log(f"[tile64] {name} M={case.M} K={case.K} N={case.N}")
    a, wp = configs.gen_a(case), configs.gen_w_packed(case)
    dwt, _ = device_convert(hr, wp)
    got = run_tile64(hr, a, dwt, case.N)
    assert hashlib.sha256(got.tobytes()).hexdigest() == digests[name]["sha256_C"], name
    del dwt, got


@pytest.mark.gpu
def test_python_host_api(oracle):
    _hr()
    rng = np.random.default_rng(11)
    a = rng.integers(-128, 128, size=(5, 256), dtype=np.int16).astype(np.int8)
    wp = oracle.pack(rng.integers(-1, 2, size=(256, 512), dtype=np.int8))
    got = tx.ternary_matmul_tile64(a, tx.interleave_tile64(wp), 512)
    np.testing.assert_array_equal(got, oracle.mm("scalar_mt", a, wp, 512))
    with pytest.raises(ValueError):
        tx.ternary_matmul_tile64(a[:, :192], tx.interleave_tile64(wp[:192]), 512)  # K % 128
