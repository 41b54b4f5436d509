"""Workspace contract of the automatic path: the size query, the caller-owned-workspace entry point
(no device allocation on the call, identical results on every planner branch, also with too little
workspace), the per-stream release, and the plan description.  Host-only checks run without a GPU
(the planner's dry run touches no device memory)."""
import ctypes

import numpy as np
import pytest

import ternixengine_amd as tx
from ternixengine_amd import hip_runtime as hr

# (M, K, N): one shape per planner branch of ternix_hip_mul_mat_ternary
BRANCH_SHAPES = [
    (1, 2560, 6912),     # M = 1: zero fill + wave GEMV whose splits add with atomics (no workspace)
    (4, 2560, 6912),     # wave GEMV, K split (in-launch sum with library workspace, reduce with caller's)
    (1, 8192, 28672),    # DMA-staged GEMV with split + reduce
    (1, 2560, 2560),     # wave GEMV, small N
    (16, 11008, 4096),   # wave GEMV, many splits + reduce
    (32, 4096, 1024),    # wave GEMV, two m-groups
    (64, 11008, 4096),   # GEMM with split-K + reduce (narrow tiles)
    (256, 16384, 1024),  # GEMM split-K, 128-row tiles
    (512, 1024, 1024),   # GEMM, no workspace
    (1, 1000, 3076),     # ragged: padded copy + wave GEMV
    (17, 4093, 1028),    # ragged: padded copy + split GEMV
    (129, 1001, 516),    # ragged: padded copy + GEMM split
    (3, 0, 64),          # K = 0
]


def describe(lib, M, K, N, a_addr=1 << 20, b_addr=1 << 24):
    buf = ctypes.create_string_buffer(192)
    st = lib.ternix_hip_plan_describe(a_addr, b_addr, M, K, N, buf, len(buf))
    return st, buf.value.decode()


def test_workspace_size_and_plan_host():
    lib = tx._load()
    sizes = {s: lib.ternix_hip_mul_mat_ternary_workspace_size(*s) for s in BRANCH_SHAPES}
    assert sizes[(512, 1024, 1024)] == 0
    assert sizes[(1, 2560, 6912)] == 0                      # M = 1: splits add into C with atomics
    assert sizes[(4, 2560, 6912)] >= 2 * 4 * 6912 * 4      # split partials of the wave GEMV
    assert sizes[(64, 11008, 4096)] >= 2 * 64 * 4096 * 4    # GEMM split partials
    assert sizes[(1, 1000, 3076)] >= 1024 * (3076 // 4)     # padded copy of W
    assert lib.ternix_hip_mul_mat_ternary_workspace_size(1, 64, 6) == 0     # rejected (N % 4)
    assert lib.ternix_hip_mul_mat_ternary_workspace_size(-1, 64, 64) == 0
    for s in BRANCH_SHAPES[:-1]:
        st, d = describe(lib, *s)
        assert st == 0 and d and d not in ("none", "rejected"), (s, d)
    assert describe(lib, 1, 2560, 6912)[1].startswith("line_gemv_kernel")
    assert describe(lib, 1, 2560, 6912, (1 << 20) + 1)[1].startswith("line_gemv_kernel ragged")  # misaligned A
    assert "pad_rows_kernel" in describe(lib, 33, 2560, 6912, (1 << 20) + 1)[1]  # 33 rows misaligned: padded
    assert describe(lib, 1, 64, 6)[0] == 1
    buf = ctypes.create_string_buffer(8)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, 1, 64, 64, buf, 0) == 1


def test_ws_entry_rejects_before_touching_pointers():
    lib = tx._load()
    # misaligned or missing workspace, bad shape: rejected before any pointer is used or work queued
    assert lib.ternix_hip_mul_mat_ternary_ws(16, 16, 16, 1, 64, 64, 17, 4096, None) == 1
    assert lib.ternix_hip_mul_mat_ternary_ws(16, 16, 16, 1, 64, 64, None, 4096, None) == 1
    assert lib.ternix_hip_mul_mat_ternary_ws(16, 16, 16, 1, 64, 6, None, 0, None) == 1


def _run_case(lib, oracle, rng, m, k, n, ws_bytes, offset=0):
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    da = hr.DeviceBuffer(max(1, a.nbytes) + 16)
    db = hr.DeviceBuffer(max(1, wp.nbytes) + 16)
    dc = hr.DeviceBuffer(4 * m * n)
    ws = hr.DeviceBuffer(max(ws_bytes, 256)) if ws_bytes else None
    if a.nbytes:
        hr.check(hr._load().hipMemcpy(ctypes.c_void_p(da.value + offset), a.ctypes.data_as(ctypes.c_void_p),
                                      a.nbytes, hr.H2D))
    if wp.nbytes:
        hr.check(hr._load().hipMemcpy(ctypes.c_void_p(db.value + offset), wp.ctypes.data_as(ctypes.c_void_p),
                                      wp.nbytes, hr.H2D))
    dc.upload(np.full(m * n, -7, np.int32))
    hr.synchronize()
    before = lib.ternix_hip_debug_alloc_count()
    st = lib.ternix_hip_mul_mat_ternary_ws(da.value + offset, db.value + offset, dc.value, m, k, n,
                                           ws.value if ws else None, ws_bytes, None)
    assert st == 0, tx.ternix_error(st)
    hr.synchronize()
    assert lib.ternix_hip_debug_alloc_count() == before, "the caller-workspace call allocated"
    got = dc.download(np.int32, (m, n))
    return got, oracle.mm("scalar_mt", a, wp, n)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", BRANCH_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_caller_workspace_every_branch(shape, oracle):
    lib = tx._load()
    m, k, n = shape
    need = lib.ternix_hip_mul_mat_ternary_workspace_size(m, k, n)
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    for ws_bytes in (need, 0):  # enough workspace: the automatic plan; none: the no-workspace plan
        print(f"shape {shape} workspace {ws_bytes} (need {need})", flush=True)
        got, ref = _run_case(lib, oracle, rng, m, k, n, ws_bytes)
        assert (got == ref).all(), (shape, ws_bytes)
    # misaligned operands: the padded-copy plans with the size the _for query gives, and the
    # generic kernels when the workspace is the aligned size only
    need_mis = lib.ternix_hip_mul_mat_ternary_workspace_size_for((1 << 20) + 3, (1 << 24) + 3, m, k, n)
    assert need_mis >= need
    for ws_bytes in (need_mis, need):
        print(f"shape {shape} misaligned, workspace {ws_bytes}", flush=True)
        got, ref = _run_case(lib, oracle, rng, m, k, n, ws_bytes, offset=3)
        assert (got == ref).all(), (shape, "misaligned", ws_bytes)


@pytest.mark.gpu
def test_release_stream_then_reuse(oracle):
    lib = tx._load()
    s = hr.Stream()
    rng = np.random.default_rng(3)
    m, k, n = 1, 2560, 6912
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n)
    ref = oracle.mm("scalar_mt", a, wp, n)
    for _ in range(2):
        assert lib.ternix_hip_mul_mat_ternary(da.value, db.value, dc.value, m, k, n, s.handle) == 0
        s.synchronize()
        assert (dc.download(np.int32, (m, n)) == ref).all()
        assert lib.ternix_hip_release_stream(s.handle) == 0
    assert lib.ternix_hip_release_stream(s.handle) == 0  # nothing left to release
