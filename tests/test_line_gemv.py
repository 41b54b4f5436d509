"""The whole-line decode GEMV (line_gemv.hip): 128-byte weight strips over a few k-steps per
workgroup, all staged at once, K splits added with int32 atomics into C that each strip's split 0
zeroes inside the launch.  Bit-exact against the CPU oracle (the reference's scalar decode, code 10
included) for every k-step count and wave form, 1 to 4 rows, a partial last strip, a partial last
split, both unit orders (split-major and the 8 XCD chunks), calls that share the strips' tickets with the other self-zeroing GEMV issued back to back,
and graph replays with eager calls between."""
import ctypes

import numpy as np
import pytest

import ternixengine_amd as tx
from ternixengine_amd import hip_runtime as hr

GARBAGE = -123456789
# (M, K, N): whole strips, a partial last strip (N/4 = 1728 = 13.5 x 128), one k-step, ragged split counts
SHAPES = [(1, 2560, 2560), (1, 2560, 6912), (1, 6912, 2560), (2, 4096, 4096), (3, 192, 1024), (4, 4160, 1536),
          (1, 64, 512), (4, 11008, 4096)]
FORMS = [(1, 8), (2, 8), (3, 8), (4, 8), (6, 8), (8, 8), (2, 4), (4, 4)]


def log(msg):
    print(msg, flush=True)


def _plan(lib, m, k, n):
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, m, k, n, buf, len(buf)) == 0
    return buf.value.decode()


def test_plan_names_line_kernel_when_forced():
    lib = tx._load()
    try:
        assert lib.ternix_hip_debug_set(b"line", 2, 8, -1, -1) == 0
        assert _plan(lib, 1, 2560, 6912).startswith("line_gemv_kernel S=2 waves=8+1 splits=20")
        assert _plan(lib, 8, 2560, 6912).startswith("line_gemv_kernel S=2")  # aligned, int32: M <= 8
        assert not _plan(lib, 9, 2560, 6912).startswith("line_gemv_kernel")
        assert _plan(lib, 1, 2560, 6900).startswith("line_gemv_kernel ragged S=2")  # N/4 % 16 != 0
        assert _plan(lib, 16, 2560, 6900).startswith("line_gemv_kernel ragged")  # ragged: more rows
        assert _plan(lib, 16, 1000, 6900).startswith("line_gemv_kernel ragged")  # 16 rows from K = 256
        assert not _plan(lib, 16, 200, 6900).startswith("line_gemv_kernel")
        assert _plan(lib, 8, 200, 6900).startswith("line_gemv_kernel ragged")  # 8 rows at any K
        assert not _plan(lib, 17, 1000, 6900).startswith("line_gemv_kernel")  # 17-32 rows from K = 1024
        assert _plan(lib, 32, 2560, 6900).startswith("line_gemv_kernel ragged")  # two 16-row groups
        assert not _plan(lib, 33, 2560, 6900).startswith("line_gemv_kernel")
        # N/4 = 224: aligned for this kernel, not for the wave kernels (N/4 % 64 != 0), whose route
        # is the padded copy: up to 16 rows here, the padded copy above
        assert _plan(lib, 16, 4864, 896).startswith("line_gemv_kernel S=2")
        assert not _plan(lib, 17, 4864, 896).startswith("line_gemv_kernel")
        assert not _plan(lib, 9, 4864, 1024).startswith("line_gemv_kernel")  # N/4 % 64 == 0: wave kernels
        assert lib.ternix_hip_debug_set(b"line", 1, 8, -1, -1) == 0
        assert not _plan(lib, 1, 8192, 4096).startswith("line_gemv_kernel")  # 128 splits > 64
    finally:
        lib.ternix_hip_debug_reset()


def _problem(oracle, rng, m, k, n):
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    return (m, k, n, hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n),
            oracle.mm("scalar_mt", a, wp, n))


def _run(p, stream=None):
    m, k, n, da, db, dc, _ = p
    kw = {} if stream is None else {"stream": stream.handle}
    assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n, **kw) == 0


def _check(p, tag):
    m, k, n, _, _, dc, expect = p
    got = dc.download(np.int32, (m, n))
    assert (got == expect).all(), (tag, m, k, n, int((got != expect).sum()))


def _reset(p):
    m, _, n, _, _, dc, _ = p
    dc.upload(np.full(m * n, GARBAGE, np.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("order", [0, 1], ids=["split_major", "xcd_chunks"])
@pytest.mark.parametrize("form", FORMS, ids=[f"S{s}_W{w}" for s, w in FORMS])
def test_line_gemv_matches_oracle(oracle, form, order):
    lib = tx._load()
    rng = np.random.default_rng(7 + form[0] * 10 + form[1])
    probs = [_problem(oracle, rng, *sh) for sh in SHAPES]
    try:
        assert lib.ternix_hip_debug_set(b"line", form[0], form[1], order, -1) == 0
        for p in probs:
            if (p[1] // 64 + form[0] - 1) // form[0] > 64:
                continue  # more than 64 splits: another plan
            log(f"[line] S={form[0]} W={form[1]} order={order} M={p[0]} K={p[1]} N={p[2]}")
            _reset(p)
            _run(p)
            hr.synchronize()
            _check(p, "first")
            _run(p)  # second call on the same tickets and outputs
            hr.synchronize()
            _check(p, "second")
    finally:
        lib.ternix_hip_debug_reset()


@pytest.mark.gpu
def test_line_gemv_interleaved_with_wave_kernel_and_graph(oracle):
    """Line-kernel calls and the wave kernel's self-zeroing calls share ticket words on one stream."""
    lib = tx._load()
    rng = np.random.default_rng(99)
    probs = [_problem(oracle, rng, *sh) for sh in [(1, 2560, 6912), (1, 6912, 2560), (4, 4096, 4096)]]
    s = hr.Stream()

    def issue_all():
        for i, p in enumerate(probs):
            lib.ternix_hip_debug_set(b"line", 2 if i != 1 else 4, 8, -1, -1)
            _run(p, s)
            lib.ternix_hip_debug_reset()  # the wave kernel's plan for the same shape and strips
            _run(p, s)

    try:
        log("[line] 200 interleaved rounds without synchronisation")
        for p in probs:
            _reset(p)
        for _ in range(200):
            issue_all()
        s.synchronize()
        for p in probs:
            _check(p, "interleaved")
        log("[line] graph replays with eager calls between")
        g = hr.Graph(s, lambda: [issue_all() for _ in range(2)])
        for rep in range(4):
            for p in probs:
                _reset(p)
            g.launch()
            s.synchronize()
            for p in probs:
                _check(p, f"replay {rep}")
            issue_all()
            s.synchronize()
            for p in probs:
                _check(p, f"eager after replay {rep}")
    finally:
        lib.ternix_hip_debug_reset()


def _line_off_and_on(lib, fn):
    """fn() with the whole-line GEMV switched off, then on (the automatic plan): both results."""
    try:
        assert lib.ternix_hip_debug_set(b"line", 0, -1, -1, -1) == 0
        off = fn()
    finally:
        lib.ternix_hip_debug_reset()
    return off, fn()


FUSED_SHAPES = [(1, 2560, 6912), (1, 6912, 2560), (2, 4096, 4096), (4, 2048, 3072), (3, 1024, 1536)]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", FUSED_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_line_gemv_dequant_and_swiglu_bit_equal(shape):
    """The float-output forms (dequantised, and dequantised + SwiGLU of interleaved column pairs)
    through the kernel's last-arriving split equal the other kernels' outputs bit for bit."""
    m, k, n = shape
    lib = tx._load()
    rng = np.random.default_rng(sum(shape))
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = (rng.integers(0, 256, size=(k, n // 4), dtype=np.uint16).astype(np.uint8) & 0x77)
    rs = rng.uniform(0.001, 0.05, size=m).astype(np.float32)
    log(f"[line dequant] M={m} K={k} N={n}")
    off, on = _line_off_and_on(lib, lambda: tx.ternary_matmul_dequant(a, wp, rs, 0.03))
    assert np.array_equal(off.view(np.int32), on.view(np.int32))
    da, db, drs = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer.from_array(rs)
    dscr = hr.DeviceBuffer(4 * m * n)

    def swiglu():
        dh = hr.DeviceBuffer(4 * m * n // 2)
        dh.upload(np.full(m * n // 2, np.nan, np.float32))
        assert lib.ternix_hip_mul_mat_ternary_swiglu(da.value, db.value, dh.value, m, k, n, drs.value, 0.03,
                                                     dscr.value, None) == 0
        hr.synchronize()
        return dh.download(np.float32, (m, n // 2))

    log(f"[line swiglu] M={m} K={k} N={n}")
    off, on = _line_off_and_on(lib, swiglu)
    assert np.isfinite(on).all() and np.array_equal(off.view(np.int32), on.view(np.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (2, 2048, 2048), (4, 1024, 2816)], ids=lambda s: "x".join(map(str, s)))
def test_line_gemv_ffn_forward_bit_equal(shape):
    """The decode feed-forward block with its two GEMVs on the whole-line kernel (RMSNorm + quantise
    fused into the gate/up GEMV, quantise into the down GEMV, dequantisation and SwiGLU in their last
    arrivers) equals the block on the other kernels bit for bit."""
    m, h, f = shape
    lib = tx._load()
    rng = np.random.default_rng(m * 7 + h)
    x = rng.standard_normal((m, h)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, size=h).astype(np.float32)
    wgu = (rng.integers(0, 256, size=(h, 2 * f // 4), dtype=np.uint16).astype(np.uint8) & 0x77)
    wd = (rng.integers(0, 256, size=(f, h // 4), dtype=np.uint16).astype(np.uint8) & 0x77)
    log(f"[line ffn] M={m} H={h} F={f}")
    off, on = _line_off_and_on(lib, lambda: tx.ffn_forward(x, g, 1e-5, wgu, 0.02, wd, 0.03))
    assert np.isfinite(on).all() and np.array_equal(off.view(np.int32), on.view(np.int32))


def _ragged_problem(oracle, rng, m, k, n, a_off, b_off):
    """Operands placed at byte offsets a_off / b_off of their buffers, the weights ending exactly at
    the end of theirs (so the kernel's last aligned dword is the buffer's last)."""
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    da = hr.DeviceBuffer(a.nbytes + a_off)
    db = hr.DeviceBuffer(wp.nbytes + b_off)
    for buf, arr, off in ((da, a, a_off), (db, wp, b_off)):
        hr.check(hr._load().hipMemcpy(ctypes.c_void_p(buf.value + off), arr.ctypes.data_as(ctypes.c_void_p),
                                      arr.nbytes, hr.H2D), "upload")
    return (m, k, n, da, db, hr.DeviceBuffer(4 * (m * n + GUARD)), oracle.mm("scalar_mt", a, wp, n), a_off, b_off)


GUARD = 1024  # int32 after C that no call may write


def _check_guarded(dc, m, n, expect, tag):
    got = dc.download(np.int32, (m * n + GUARD,))
    assert (got[m * n:] == GARBAGE).all(), (tag, "guard region written")
    got = got[:m * n].reshape(m, n)
    assert (got == expect).all(), (tag, int((got != expect).sum()))


# (M, K, N, A offset, W offset): the ragged configurations, K < 64, one byte per row, odd row lengths,
# misaligned operands on aligned shapes, a partial last 16-byte group
RAGGED = [(1, 1000, 3076, 0, 0), (4, 1000, 3076, 0, 0), (2, 4093, 1028, 0, 0), (3, 37, 20, 0, 0),
          (1, 5, 4, 0, 0), (2, 777, 516, 3, 1), (4, 4096, 1024, 3, 0), (1, 2560, 6912, 0, 2),
          (3, 130, 2044, 1, 3), (1, 8191, 2052, 0, 0), (12, 1500, 3076, 0, 0), (16, 4093, 1028, 2, 1),
          (17, 4093, 1028, 0, 0), (24, 2000, 1036, 1, 2), (32, 1500, 516, 0, 0),
          (1, 16, 4, 0, 1), (2, 9, 8, 1, 3)]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", RAGGED, ids=lambda s: "x".join(map(str, s)))
def test_line_gemv_ragged_matches_oracle(oracle, shape):
    """Ragged and misaligned operands go to the whole-line GEMV's register-staged form (no padded
    copy; 17-32 rows in two 16-row groups): bit-exact against the oracle, twice in a row on the same
    tickets, and in graph replays (operands of 5 to 18 bytes take the loads near the operands' end)."""
    lib = tx._load()
    m, k, n, ao, bo = shape
    p = _ragged_problem(oracle, np.random.default_rng(sum(shape)), *shape)
    _, _, _, da, db, dc, expect, _, _ = p
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe((1 << 20) + ao, (1 << 24) + bo, m, k, n, buf, len(buf)) == 0
    # two row groups take the ragged form on 64 workgroups or more (2 k-steps each here), else the
    # padded copy
    strips, splits = -(-(n // 4) // 128), -(-(-(-k // 64)) // 2)
    want = "pad_rows_kernel" if m > 16 and strips * splits < 64 else "line_gemv_kernel ragged"
    assert buf.value.decode().startswith(want), buf.value
    s = hr.Stream()
    call = lambda: tx.mul_mat_ternary(da.value + ao, db.value + bo, dc.value, m, k, n, stream=s.handle)
    log(f"[line ragged] M={m} K={k} N={n} A+{ao} W+{bo}")
    for rep in range(2):
        dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
        assert call() == 0
        s.synchronize()
        _check_guarded(dc, m, n, expect, rep)
    g = hr.Graph(s, call)
    for rep in range(3):
        dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
        g.launch()
        s.synchronize()
        _check_guarded(dc, m, n, expect, ("replay", rep))
        assert call() == 0
        s.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(5, 4096, 11008), (6, 2560, 6912), (7, 192, 1024), (8, 11008, 4096)],
                         ids=lambda s: "x".join(map(str, s)))
def test_line_gemv_five_to_eight_rows(oracle, shape):
    """Aligned operands with 5-8 rows and an int32 output take the whole-line GEMV on the automatic
    plan: bit-exact against the oracle on two calls in a row."""
    lib = tx._load()
    m, k, n = shape
    p = _ragged_problem(oracle, np.random.default_rng(sum(shape) + 5), m, k, n, 0, 0)
    _, _, _, da, db, dc, expect, _, _ = p
    assert _plan(lib, m, k, n).startswith("line_gemv_kernel S="), _plan(lib, m, k, n)
    log(f"[line 5-8 rows] M={m} K={k} N={n}")
    for rep in range(2):
        dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
        hr.synchronize()
        _check_guarded(dc, m, n, expect, rep)


@pytest.mark.gpu
def test_line_gemv_random_ragged_offsets(oracle):
    """Seeded random ragged shapes up to 32 rows with A and W at random byte offsets, each operand
    ending exactly at the end of its buffer, on the automatic path: bit-exact against the oracle,
    nothing written past C."""
    rng = np.random.default_rng(909)
    s = hr.Stream()
    for t in range(30):
        m = int(rng.integers(1, 33))
        k = int(rng.integers(1, 3000))
        n = 4 * int(rng.integers(1, 800))
        ao, bo = int(rng.integers(0, 16)), int(rng.integers(0, 16))
        p = _ragged_problem(oracle, np.random.default_rng(t), m, k, n, ao, bo)
        _, _, _, da, db, dc, expect, _, _ = p
        log(f"[line random offsets] trial {t} M={m} K={k} N={n} A+{ao} W+{bo}")
        dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
        assert tx.mul_mat_ternary(da.value + ao, db.value + bo, dc.value, m, k, n, stream=s.handle) == 0
        s.synchronize()
        _check_guarded(dc, m, n, expect, t)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 4])
def test_line_gemv_two_workgroups_per_cu(oracle, m):
    """8192 x 8192 on the automatic plan: 16 strips x 32 splits of 4 k-steps, two workgroups per CU
    (preferred to 16 splits of 8 k-steps on one), bit-exact against the oracle on two calls."""
    lib = tx._load()
    k = n = 8192
    p = _ragged_problem(oracle, np.random.default_rng(8192 + m), m, k, n, 0, 0)
    _, _, _, da, db, dc, expect, _, _ = p
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, m, k, n, buf, len(buf)) == 0
    plan = buf.value.decode()
    if hr.device_attribute(hr.ATTR_MULTIPROCESSOR_COUNT) == 256:
        assert plan.startswith("line_gemv_kernel S=4 waves=8+1 splits=32"), plan
    log(f"[line two per CU] M={m} K={k} N={n} plan={plan[:40]}")
    for rep in range(2):
        dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
        hr.synchronize()
        _check_guarded(dc, m, n, expect, rep)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(5, 2560, 6912), (8, 4096, 4096), (16, 2560, 2560), (16, 6912, 2560),
                                   (12, 1000, 3076), (7, 64, 512)], ids=lambda s: "x".join(map(str, s)))
def test_line_gemv_up_to_16_rows(oracle, shape):
    """With the row limit raised to 16, 5-16 rows run through the whole-line GEMV (every lane group's
    rows in the epilogue), aligned and ragged, bit-exact against the oracle."""
    lib = tx._load()
    m, k, n = shape
    p = _ragged_problem(oracle, np.random.default_rng(sum(shape)), m, k, n, 0, 0)
    _, _, _, da, db, dc, expect, _, _ = p
    try:
        assert lib.ternix_hip_debug_set(b"line", -1, -1, -1, 16) == 0
        buf = ctypes.create_string_buffer(192)
        assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, m, k, n, buf, len(buf)) == 0
        assert buf.value.decode().startswith("line_gemv_kernel"), buf.value
        log(f"[line 16 rows] M={m} K={k} N={n}")
        for rep in range(2):
            dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
            assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
            hr.synchronize()
            _check_guarded(dc, m, n, expect, rep)
    finally:
        lib.ternix_hip_debug_reset()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 2560, 6912), (2, 2048, 2048), (4, 1024, 2816), (1, 1024, 16384), (3, 512, 640),
                                   (1, 512, 20480), (2, 4096, 2048)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("zero_x", [False, True], ids=["x", "x0"])
def test_line_gemv_ffn_strip_maxima_bit_equal(shape, zero_x):
    """The decode block's down GEMV quantising h from the gate/up launch's per-strip maxima equals the
    same block with the down GEMV reading whole rows of h (and the block on the other kernels) bit for
    bit; an all-zero x gives all-zero h, whose absmax is the 1e-5 floor."""
    m, h, f = shape
    lib = tx._load()
    rng = np.random.default_rng(m * 11 + f)
    x = np.zeros((m, h), np.float32) if zero_x else rng.standard_normal((m, h)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, size=h).astype(np.float32)
    wgu = (rng.integers(0, 256, size=(h, 2 * f // 4), dtype=np.uint16).astype(np.uint8) & 0x77)
    wd = (rng.integers(0, 256, size=(f, h // 4), dtype=np.uint16).astype(np.uint8) & 0x77)
    run = lambda: tx.ffn_forward(x, g, 1e-5, wgu, 0.02, wd, 0.03)
    log(f"[line ffn maxima] M={m} H={h} F={f} zero_x={zero_x}")
    try:
        assert lib.ternix_hip_debug_set(b"ffn_amax", 0, -1, -1, -1) == 0
        rows = run()
    finally:
        lib.ternix_hip_debug_reset()
    maxima = run()
    off, _ = _line_off_and_on(lib, run)
    assert np.isfinite(maxima).all()
    assert np.array_equal(rows.view(np.int32), maxima.view(np.int32))
    assert np.array_equal(off.view(np.int32), maxima.view(np.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(9, 4864, 896), (16, 2432, 896), (16, 8192, 896), (12, 130, 448)],
                         ids=lambda s: "x".join(map(str, s)))
def test_line_gemv_rows_instead_of_padded_copy(oracle, shape):
    """Operands aligned for the whole-line GEMV but not for the wave kernels (N/4 % 64 != 0) take the
    whole-line GEMV up to 16 rows (8 below K = 256) instead of the padded copy: bit-exact against
    the oracle on two calls in a row."""
    lib = tx._load()
    m, k, n = shape
    p = _ragged_problem(oracle, np.random.default_rng(sum(shape) + 11), m, k, n, 0, 0)
    _, _, _, da, db, dc, expect, _, _ = p
    plan = _plan(lib, m, k, n)
    assert plan.startswith("line_gemv_kernel S=") == (k >= 256), plan
    log(f"[line instead of padded copy] M={m} K={k} N={n} plan={plan[:40]}")
    for rep in range(2):
        dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
        hr.synchronize()
        _check_guarded(dc, m, n, expect, rep)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,s", [((1, 8192, 1024), 4), ((1, 4096, 4096), 3), ((8, 2560, 6912), 4),
                                     ((1, 2560, 6912), 3), ((4, 6912, 2560), 4), ((1, 4096, 1024), 3)],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else f"S{v}")
def test_line_gemv_minimum_k_steps(oracle, shape, s):
    """The automatic plan's k-steps per workgroup: at least 3 from 64 k-steps, 4 from 96 and 4 with
    5-8 rows from 40 (a 256-CU device), bit-exact against the oracle."""
    lib = tx._load()
    m, k, n = shape
    p = _ragged_problem(oracle, np.random.default_rng(sum(shape) + 13), m, k, n, 0, 0)
    _, _, _, da, db, dc, expect, _, _ = p
    plan = _plan(lib, m, k, n)
    if hr.device_attribute(hr.ATTR_MULTIPROCESSOR_COUNT) == 256:
        assert plan.startswith(f"line_gemv_kernel S={s} "), plan
    log(f"[line minimum k-steps] M={m} K={k} N={n} plan={plan[:40]}")
    dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
    assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
    hr.synchronize()
    _check_guarded(dc, m, n, expect, 0)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,line", [((8, 8192, 8192), False), ((7, 14336, 4096), False), ((8, 11008, 4096), True),
                                        ((6, 8192, 8192), True)], ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_line_gemv_seven_eight_rows_one_per_cu(oracle, shape, line):
    """7-8 rows on aligned operands: the whole-line GEMV only with one workgroup per CU, else the
    wave-pipelined kernel (plans on a 256-CU device); bit-exact against the oracle."""
    lib = tx._load()
    m, k, n = shape
    p = _ragged_problem(oracle, np.random.default_rng(sum(shape) + 17), m, k, n, 0, 0)
    _, _, _, da, db, dc, expect, _, _ = p
    plan = _plan(lib, m, k, n)
    if hr.device_attribute(hr.ATTR_MULTIPROCESSOR_COUNT) == 256:
        assert plan.startswith("line_gemv_kernel S=") == line, plan
    log(f"[line 7-8 rows] M={m} K={k} N={n} plan={plan[:40]}")
    dc.upload(np.full(m * n + GUARD, GARBAGE, np.int32))
    assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n) == 0
    hr.synchronize()
    _check_guarded(dc, m, n, expect, 0)
