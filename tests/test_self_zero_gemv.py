"""The M = 1 split-K GEMV whose splits add into C with int32 atomics, C being zeroed inside the same
launch by each strip's first split (per-strip ticket counters and "zeroed" words that persist across
calls, one block of 64 tickets per call): bit-exact for calls of different shapes and split counts
that share the strips' tickets, issued back to back without synchronisation, replayed from a
hipGraph with eager calls in between, and on two streams at once."""
import ctypes

import numpy as np
import pytest

import ternixengine_amd as tx
from ternixengine_amd import hip_runtime as hr

GARBAGE = -123456789
# (K, N): 16-byte strips with 6 splits, 32-byte strips with 4 and 10 splits, a 1024-wide strip count
SHAPES = [(2560, 2560), (2560, 6912), (6912, 2560), (4096, 4096), (1024, 2048)]


def _debug_reset(lib):
    """Every switch off, and the whole-line GEMV (which takes most M <= 4 shapes first) off too: these
    tests cover the wave-pipelined and DMA-staged kernels' self-zeroing plans."""
    lib.ternix_hip_debug_reset()
    assert lib.ternix_hip_debug_set(b"line", 0, -1, -1, -1) == 0


@pytest.fixture(autouse=True)
def _no_line_kernel():
    lib = tx._load()
    _debug_reset(lib)
    yield
    lib.ternix_hip_debug_reset()


def log(msg):
    print(msg, flush=True)


def _plan(lib, k, n):
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, 1, k, n, buf, len(buf)) == 0
    return buf.value.decode()


def test_plan_names_self_zeroing():
    lib = tx._load()
    _debug_reset(lib)
    for k, n in SHAPES[:3]:
        assert "zeroed by each strip's first split" in _plan(lib, k, n), (k, n)
    assert lib.ternix_hip_debug_set(b"self_zero", 0, -1, -1, -1) == 0
    try:
        assert _plan(lib, 2560, 6912).startswith("zero_kernel + ")
    finally:
        _debug_reset(lib)


# tile-64 weights: K > 4096 takes the split wave kernel (the shorter K the whole-K kernel)
TILE64_SHAPES = [(6912, 2560), (8192, 1024)]


def _problems(oracle, seed):
    rng = np.random.default_rng(seed)
    out = []
    for (k, n), path in [(s, "auto") for s in SHAPES] + [(s, "tile64") for s in TILE64_SHAPES]:
        a = rng.integers(-128, 128, size=(1, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        expect = oracle.mm("scalar_mt", a, wp, n)
        w_dev = tx.interleave_tile64(wp) if path == "tile64" else wp
        out.append((k, n, path, hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(w_dev),
                    hr.DeviceBuffer(4 * n), expect))
    return out


def _issue(probs, s):
    for k, n, path, da, db, dc, _ in probs:
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, 1, k, n, stream=s.handle, path=path) == 0


def _check(probs, tag):
    for k, n, path, _, _, dc, expect in probs:
        assert (dc.download(np.int32, (1, n)) == expect).all(), (tag, k, n, path)


def _reset(probs):
    for _, n, _, _, _, dc, _ in probs:
        dc.upload(np.full(n, GARBAGE, np.int32))


@pytest.mark.gpu
def test_self_zero_interleaved_and_graph(oracle):
    s = hr.Stream()
    probs = _problems(oracle, 41)
    log("[self-zero] one call each")
    _reset(probs)
    _issue(probs, s)
    s.synchronize()
    _check(probs, "first")
    log("[self-zero] 300 interleaved rounds without synchronisation")
    _reset(probs)
    for _ in range(300):
        _issue(probs, s)
    s.synchronize()
    _check(probs, "interleaved")
    log("[self-zero] graph replays with eager calls between")
    g = hr.Graph(s, lambda: [_issue(probs, s) for _ in range(3)])
    for rep in range(5):
        _reset(probs)
        g.launch()
        s.synchronize()
        _check(probs, f"replay {rep}")
        _reset(probs)
        _issue(probs, s)
        s.synchronize()
        _check(probs, f"eager after replay {rep}")


@pytest.mark.gpu
def test_self_zero_two_streams(oracle):
    s1, s2 = hr.Stream(), hr.Stream()
    p1, p2 = _problems(oracle, 42), _problems(oracle, 43)
    _reset(p1)
    _reset(p2)
    log("[self-zero] two streams, 100 rounds each")
    for _ in range(100):
        _issue(p1, s1)
        _issue(p2, s2)
    s1.synchronize()
    s2.synchronize()
    _check(p1, "stream 1")
    _check(p2, "stream 2")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [2, 3, 4])
def test_self_zero_few_rows(oracle, m):
    """2..4 rows take the same plans (wave kernel with 32-byte strips, DMA kernel on wide matrices):
    interleaved calls of three shapes, every row bit-exact."""
    lib = tx._load()
    _debug_reset(lib)
    s = hr.Stream()
    rng = np.random.default_rng(50 + m)
    probs = []
    for k, n in [(4096, 11008), (11008, 4096), (8192, 28672)]:
        plan = _plan_m(lib, m, k, n)
        assert "zeroed by each strip's first split" in plan, plan
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        probs.append((m, k, n, hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp),
                      hr.DeviceBuffer(4 * m * n), oracle.mm("scalar_mt", a, wp, n)))
    for _, _, n, _, _, dc, _ in probs:
        dc.upload(np.full(m * n, GARBAGE, np.int32))
    log(f"[self-zero M={m}] 30 interleaved rounds")
    for _ in range(30):
        for mm, k, n, da, db, dc, _ in probs:
            assert tx.mul_mat_ternary(da.value, db.value, dc.value, mm, k, n, stream=s.handle) == 0
    s.synchronize()
    for mm, k, n, _, _, dc, expect in probs:
        assert (dc.download(np.int32, (mm, n)) == expect).all(), (mm, k, n)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [5, 8, 16])
def test_self_zero_up_to_16_rows(oracle, m):
    """5..16 rows take the same plan with the 16-row coalesced atomic epilogue: interleaved calls of
    three shapes on one stream, then the same calls with the plan limited to 4 rows (in-launch sums
    and the reduce launch) on the same output buffers, every row bit-exact."""
    lib = tx._load()
    _debug_reset(lib)
    s = hr.Stream()
    rng = np.random.default_rng(60 + m)
    probs = []
    for k, n in [(4096, 11008), (11008, 4096), (2560, 6912)]:
        plan = _plan_m(lib, m, k, n)
        assert "zeroed by each strip's first split" in plan, plan
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        probs.append((m, k, n, hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp),
                      hr.DeviceBuffer(4 * m * n), oracle.mm("scalar_mt", a, wp, n)))
    try:
        for limit in (-1, 4):
            assert lib.ternix_hip_debug_set(b"m1_atomic", -1, limit, -1, -1) == 0
            for _, _, n, _, _, dc, _ in probs:
                dc.upload(np.full(m * n, GARBAGE, np.int32))
            log(f"[self-zero M={m} row limit {limit}] 30 interleaved rounds")
            for _ in range(30):
                for mm, k, n, da, db, dc, _ in probs:
                    assert tx.mul_mat_ternary(da.value, db.value, dc.value, mm, k, n, stream=s.handle) == 0
            s.synchronize()
            for mm, k, n, _, _, dc, expect in probs:
                assert (dc.download(np.int32, (mm, n)) == expect).all(), (mm, k, n, limit)
    finally:
        _debug_reset(lib)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [17, 24, 32, 64])
def test_self_zero_several_m_groups(oracle, m):
    """Above 16 rows the plan runs one 16-row m-group per workgroup row of the grid, with one ticket
    pair per (m-group, strip): interleaved calls of two shapes with several m-groups, bit-exact, then
    the same calls with the plan limited to 16 rows on the same output buffers."""
    lib = tx._load()
    _debug_reset(lib)
    s = hr.Stream()
    rng = np.random.default_rng(80 + m)
    probs = []
    for k, n in [(4096, 4096), (6912, 2560)]:
        plan = _plan_m(lib, m, k, n)
        assert "zeroed by each strip's first split" in plan, (m, k, n, plan)
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        probs.append((m, k, n, hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp),
                      hr.DeviceBuffer(4 * m * n), oracle.mm("scalar_mt", a, wp, n)))
    try:
        for limit in (-1, 16):
            assert lib.ternix_hip_debug_set(b"m1_atomic", -1, limit, -1, -1) == 0
            for _, _, n, _, _, dc, _ in probs:
                dc.upload(np.full(m * n, GARBAGE, np.int32))
            log(f"[self-zero M={m} row limit {limit}] 30 interleaved rounds")
            for _ in range(30):
                for mm, k, n, da, db, dc, _ in probs:
                    assert tx.mul_mat_ternary(da.value, db.value, dc.value, mm, k, n, stream=s.handle) == 0
            s.synchronize()
            for mm, k, n, _, _, dc, expect in probs:
                assert (dc.download(np.int32, (mm, n)) == expect).all(), (mm, k, n, limit)
    finally:
        _debug_reset(lib)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [4, 16])
def test_self_zero_tile64_rows(oracle, m):
    """Tile-64 weights with K > 4096 take the atomic plan for up to 16 rows too: interleaved calls of
    two shapes, bit-exact, then the reduce plan (row limit 1) on the same buffers."""
    lib = tx._load()
    _debug_reset(lib)
    s = hr.Stream()
    rng = np.random.default_rng(70 + m)
    probs = []
    for k, n in [(11008, 4096), (6912, 2560)]:
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        probs.append((m, k, n, hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(tx.interleave_tile64(wp)),
                      hr.DeviceBuffer(4 * m * n), oracle.mm("scalar_mt", a, wp, n)))
    try:
        for limit in (-1, 1):
            assert lib.ternix_hip_debug_set(b"m1_atomic", -1, -1, limit, -1) == 0
            for _, _, n, _, _, dc, _ in probs:
                dc.upload(np.full(m * n, GARBAGE, np.int32))
            log(f"[self-zero tile-64 M={m} row limit {limit}] 30 interleaved rounds")
            for _ in range(30):
                for mm, k, n, da, db, dc, _ in probs:
                    assert tx.mul_mat_ternary(da.value, db.value, dc.value, mm, k, n, stream=s.handle,
                                              path="tile64") == 0
            s.synchronize()
            for mm, k, n, _, _, dc, expect in probs:
                assert (dc.download(np.int32, (mm, n)) == expect).all(), (mm, k, n, limit)
    finally:
        _debug_reset(lib)


def _plan_m(lib, m, k, n):
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, m, k, n, buf, len(buf)) == 0
    return buf.value.decode()


@pytest.mark.gpu
def test_self_zero_dma_kernel(oracle):
    """The DMA-staged kernel's form of the same plan (wide M = 1 GEMVs): repeated calls of two
    shapes sharing the strips' tickets, then the reduce plan (self_zero off) on the same buffers."""
    lib = tx._load()
    _debug_reset(lib)
    assert lib.ternix_hip_debug_set(b"self_zero", 2, -1, -1, -1) == 0
    try:
        s = hr.Stream()
        rng = np.random.default_rng(44)
        probs = []
        for k, n in [(8192, 28672), (4096, 16384)]:
            assert "skinny_dma_kernel" in _plan(lib, k, n) and "zeroed" in _plan(lib, k, n), _plan(lib, k, n)
            a = rng.integers(-128, 128, size=(1, k), dtype=np.int8)
            wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
            probs.append((k, n, "auto", hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp),
                          hr.DeviceBuffer(4 * n), oracle.mm("scalar_mt", a, wp, n)))
        log("[self-zero dma] 50 interleaved rounds")
        _reset(probs)
        for _ in range(50):
            _issue(probs, s)
        s.synchronize()
        _check(probs, "dma interleaved")
        assert lib.ternix_hip_debug_set(b"self_zero", 0, -1, -1, -1) == 0
        assert "splitk_reduce_kernel" in _plan(lib, 8192, 28672)
        _reset(probs)
        _issue(probs, s)
        s.synchronize()
        _check(probs, "reduce plan after")
    finally:
        _debug_reset(lib)


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(1, 1000, 3076), (3, 2000, 1036), (17, 4093, 1028), (32, 1000, 516)])
def test_self_zero_padded_real_columns(oracle, m, k, n):
    """Ragged shapes run the atomic plan on padded copies and write only the N real columns of C at
    pitch N: a guard region after C keeps its values, and C is bit-exact over repeated calls, two
    of them back to back without synchronisation."""
    lib = tx._load()
    _debug_reset(lib)
    plan = _plan_m(lib, m, k, n)
    assert plan.startswith("pad_rows_kernel + skinny_wave_kernel") and "zeroed by each strip's first split" in plan, plan
    rng = np.random.default_rng(1000 + m)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    expect = oracle.mm("scalar_mt", a, wp, n)
    guard = 4096
    da, db = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp)
    dc = hr.DeviceBuffer(4 * (m * n + guard))
    dc.upload(np.full(m * n + guard, GARBAGE, np.int32))
    log(f"[self-zero padded] M={m} K={k} N={n}")
    for _ in range(3):
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
    hr.synchronize()
    got = dc.download(np.int32, (m * n + guard,))
    assert (got[: m * n].reshape(m, n) == expect).all(), (m, k, n)
    assert (got[m * n:] == GARBAGE).all(), (m, k, n)


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(1, 192, 4096), (1, 128, 16384), (3, 192, 8192), (1, 320, 2048), (16, 192, 4096)])
def test_self_zero_short_k_ranges(oracle, m, k, n):
    """Splits of one to three k-steps, so some of a workgroup's four waves own no step at all (each
    wave issues only its own steps): bit-exact over repeated calls."""
    lib = tx._load()
    _debug_reset(lib)
    plan = _plan_m(lib, m, k, n)
    rng = np.random.default_rng(2000 + k + m)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    expect = oracle.mm("scalar_mt", a, wp, n)
    da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n)
    dc.upload(np.full(m * n, GARBAGE, np.int32))
    log(f"[short k-ranges] M={m} K={k} N={n}: {plan}")
    for _ in range(3):
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
    hr.synchronize()
    assert (dc.download(np.int32, (m, n)) == expect).all(), (m, k, n, plan)


def test_plan_column_waves():
    """The M <= 4 atomic plan takes column waves where one round of workgroups needs at most 32
    splits (cfg3 M=4, cfg2 up), not for cfg2 down (5 strips), cfg1 (16-byte strips) or M = 16, and
    the switch forces them off."""
    lib = tx._load()
    _debug_reset(lib)
    for m, k, n in [(4, 4096, 11008), (4, 11008, 4096), (1, 2560, 6912)]:
        assert "column waves" in _plan_m(lib, m, k, n), (m, k, n)
    for m, k, n in [(1, 6912, 2560), (1, 2560, 2560), (16, 4096, 11008)]:
        assert "column waves" not in _plan_m(lib, m, k, n), (m, k, n)
    assert lib.ternix_hip_debug_set(b"wave_sw", -1, -1, 0, -1) == 0
    try:
        assert "column waves" not in _plan_m(lib, 4, 4096, 11008)
    finally:
        _debug_reset(lib)
