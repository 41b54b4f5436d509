"""HIP-vs-CPU bit-exact suite (replaces the reference's tests/test_cuda_matmul.cu).

Every kernel path is called through the C-ABI (include/ternix/ternix_hip.h) on device buffers and
compared for exact int32 equality with
  * the golden vectors written by the reference's compiled CPU code (tests/golden/),
  * the CPU oracle (oracle/) on the same seeded inputs, at sizes it finishes in seconds,
  * the SHA-256 digests of the reference's outputs for every benchmark configuration at full size,
  * closed forms (worst-case magnitude, W == 0, W == +1, identity).
C is prefilled with garbage before each call, so cells a kernel fails to write are caught
(reference tests/test_cuda_matmul.cu:20,23)."""
import ctypes
import hashlib
import sys

import numpy as np
import pytest

from conftest import small_case_list

pytestmark = pytest.mark.gpu

import ternixengine_amd as tx  # noqa: E402
from ternixengine_amd import configs  # noqa: E402
from ternixengine_amd import hip_runtime as hr  # noqa: E402

PATHS = ["auto", "gemv", "gemm", "naive", "tiled"]
GARBAGE = np.int32(-0x2A2A2A2B)


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if hr.device_count() < 1:
        pytest.skip("no HIP device")
    tx._load()
    yield
    hr.synchronize()


def supports(path, m, k, n):
    if path == "gemv":
        return m <= 32
    if path == "tiled":
        return m % 64 == 0 and n % 64 == 0 and k % 64 == 0
    if path == "naive":
        return m * n * k <= 1 << 28
    return True


def run(path, a, wp, n, a_off=0, b_off=0, c_off=0, stream=None):
    """C = A x W on the GPU through the C-ABI; optional byte offsets misalign the pointers."""
    a = np.ascontiguousarray(a, np.int8)
    wp = np.ascontiguousarray(wp, np.uint8)
    m, k = a.shape
    da = hr.DeviceBuffer(a.nbytes + 64)
    db = hr.DeviceBuffer(wp.nbytes + 64)
    dc = hr.DeviceBuffer(4 * m * n + 64)
    pa, pb, pc = da.value + a_off, db.value + b_off, dc.value + c_off
    if a.nbytes:
        hr.check(hr._load().hipMemcpy(ctypes.c_void_p(pa), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, hr.H2D), "A")
    if wp.nbytes:
        hr.check(hr._load().hipMemcpy(ctypes.c_void_p(pb), wp.ctypes.data_as(ctypes.c_void_p), wp.nbytes, hr.H2D), "B")
    garbage = np.full(m * n + 16, GARBAGE, np.int32)
    dc.upload(garbage)
    st = tx.mul_mat_ternary(pa, pb, pc, m, k, n, stream=stream.handle if stream else None, path=path)
    assert st == 0, f"{path} returned {st} ({tx.ternix_error(st)})"
    hr.synchronize()
    out = np.empty((m, n), np.int32)
    if out.nbytes:
        hr.check(hr._load().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(pc), out.nbytes, hr.D2H),
                 "C")
    return out


@pytest.mark.parametrize("path", PATHS)
def test_reference_suite_shapes(golden, path):
    for m, k, n, i in small_case_list(golden):
        if not supports(path, m, k, n):
            continue
        log(f"[{path}] golden case {i} M={m} K={k} N={n}")
        got = run(path, golden[f"s{i}_A"], golden[f"s{i}_Wp"], n)
        assert (got == golden[f"s{i}_C"]).all(), (path, m, k, n)


@pytest.mark.parametrize("path", ["auto", "gemv", "gemm", "naive"])
def test_out_of_domain_code_matches_reference_scalar(golden, path):
    # code 10 decodes as -2, like reference mul_mat_ternary_scalar and the CUDA decode2.
    log(f"[{path}] out-of-domain code")
    got = run(path, golden["invalid_A"], golden["invalid_Wp"], golden["invalid_C_scalar"].shape[1])
    assert (got == golden["invalid_C_scalar"]).all()


@pytest.mark.parametrize("path", ["auto", "gemv", "gemm"])
def test_extreme_activations(golden, path):
    log(f"[{path}] extreme activations")
    got = run(path, golden["extreme_A"], golden["extreme_Wp"], 16)
    assert (got == golden["extreme_C"]).all()


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_closed_forms(oracle, path):
    rng = np.random.default_rng(2)
    for m, k, n in ((1, 320, 64), (7, 1000, 1028), (20, 130, 260)):
        log(f"[{path}] closed forms M={m} K={k} N={n}")
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        assert (run(path, a, oracle.pack(np.zeros((k, n), np.int8)), n) == 0).all()
        rs = a.astype(np.int64).sum(axis=1)
        assert (run(path, a, oracle.pack(np.ones((k, n), np.int8)), n) == rs[:, None]).all()
        worst = np.full((m, k), -128, np.int8)
        assert (run(path, worst, oracle.pack(-np.ones((k, n), np.int8)), n) == 128 * k).all()
    eye = np.eye(256, dtype=np.int8)
    a = rng.integers(-128, 128, size=(9, 256), dtype=np.int8)
    assert (run(path, a, oracle.pack(eye), 256) == a.astype(np.int32)).all()


@pytest.mark.parametrize("path", ["auto", "gemv", "gemm", "naive"])
def test_random_ragged_shapes(oracle, path):
    rng = np.random.default_rng(17)
    for trial in range(24):
        m = int(rng.integers(1, 33 if path == "gemv" else 150))
        k = int(rng.integers(0, 700))
        n = 4 * int(rng.integers(1, 300))
        log(f"[{path}] ragged trial {trial} M={m} K={k} N={n}")
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        expect = oracle.mm("scalar", a, wp, n)
        assert (run(path, a, wp, n) == expect).all(), (m, k, n)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_misaligned_pointers(oracle, path):
    rng = np.random.default_rng(23)
    for (m, k, n), (ao, bo, co) in (((3, 256, 512), (1, 3, 4)), ((40 if path == "gemm" else 30, 512, 1024), (5, 2, 8)),
                                    ((2, 64, 64), (16, 4, 16))):
        log(f"[{path}] misaligned M={m} K={k} N={n} offsets A+{ao} B+{bo} C+{co}")
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        assert (run(path, a, wp, n, ao, bo, co) == oracle.mm("scalar", a, wp, n)).all()


def test_k_beyond_accumulator_bound(oracle):
    # K > 2^17 forces the launch layer to split K (scaled partial sums stay exact); the largest
    # in-domain term is -128 * -1 per row, so a single unsplit accumulator would overflow here.
    m, k, n = 2, (1 << 18) + 200, 16
    a = np.full((m, k), -128, np.int8)
    a[1, ::3] = 127
    w = -np.ones((k, n), np.int8)
    w[:, 5] = 1
    wp = oracle.pack(w)
    expect = (a.astype(np.int64) @ w.astype(np.int64))
    assert np.abs(expect).max() < 2 ** 31
    for path in ("gemv", "gemm"):
        log(f"[{path}] K={k}")
        assert (run(path, a, wp, n) == expect).all(), path
    # out-of-domain code 10 everywhere (reference scalar decode: -2 per weight) just above 2^17 rows
    k = (1 << 17) + 100
    a = np.full((m, k), -128, np.int8)
    wp = np.full((k, n // 4), 0xAA, np.uint8)
    for path in ("gemv", "gemm"):
        log(f"[{path}] K={k} code 10")
        assert (run(path, a, wp, n) == 256 * k).all(), path


def test_k_zero_writes_zeros():
    for path in ("auto", "gemv", "gemm", "naive"):
        got = run(path, np.zeros((3, 0), np.int8), np.zeros((0, 8), np.uint8), 32)
        assert (got == 0).all(), path


def test_on_user_stream(oracle):
    s = hr.Stream()
    rng = np.random.default_rng(4)
    a = rng.integers(-128, 128, size=(4, 640), dtype=np.int8)
    wp = rng.integers(0, 256, size=(640, 96), dtype=np.uint8)
    assert (run("auto", a, wp, 384, stream=s) == oracle.mm("scalar", a, wp, 384)).all()


def test_host_wrapper_and_python_api(oracle, golden):
    for m, k, n, i in small_case_list(golden):
        for impl in ("hip", "hip_gemm", "hip_naive") + (("hip_gemv",) if m <= 32 else ()):
            got = tx.ternary_matmul(golden[f"s{i}_A"], golden[f"s{i}_Wp"], impl)
            assert (got == golden[f"s{i}_C"]).all(), (impl, m, k, n)
    # reference tests/test_python_binding.py:35-39 shape through the tiled contract
    rng = np.random.default_rng(3)
    a = rng.integers(-128, 128, size=(128, 256), dtype=np.int8)
    w = rng.integers(-1, 2, size=(256, 192), dtype=np.int8)
    assert (tx.ternary_matmul(a, tx.pack_ternary(w), "hip_tiled") == a.astype(np.int32) @ w.astype(np.int32)).all()
    with pytest.raises(RuntimeError, match="HIP error"):
        tx.ternary_matmul(a[:65], tx.pack_ternary(w), "hip_tiled")


ORACLE_CASES = ["cfg1", "cfg2_up", "cfg2_down", "cfg3_m4_up", "cfg3_m4_down", "cfg3_m16_up", "cfg3_m16_down",
                "cfg3_m64_up", "cfg3_m64_down", "cfg5_ragged_1x1000x3076", "cfg5_ragged_17x4093x1028",
                "cfg5_ragged_129x8191x2052", "cfg5_big_m1"]


@pytest.mark.parametrize("name", ORACLE_CASES)
def test_config_against_oracle(oracle, digests, name):
    case = configs.CASES[name]
    a, wp = configs.gen_a(case), configs.gen_w_packed(case)
    expect = oracle.mm("scalar_mt", a, wp, case.N)
    for path in ("auto", "gemv", "gemm"):
        if not supports(path, case.M, case.K, case.N):
            continue
        log(f"[{path}] {name} M={case.M} K={case.K} N={case.N}")
        got = run(path, a, wp, case.N)
        assert (got == expect).all(), (path, name)
        assert hashlib.sha256(got.tobytes()).hexdigest() == digests[name]["sha256_C"]


FULL_CASES = ["cfg4_4096x4096", "cfg4_4096x14336", "cfg4_14336x4096", "cfg5_big_m4096", "cfg5_worst",
              "refbench_n512", "refbench_n1024", "refbench_n2048", "refbench_n4096"]


@pytest.mark.parametrize("name", FULL_CASES)
def test_config_full_size_digest(digests, name):
    """Full-size MFMA configurations: bit-exact via the SHA-256 of the reference avx2_blocked output."""
    case = configs.CASES[name]
    a, wp = configs.gen_a(case), configs.gen_w_packed(case)
    d = digests[name]
    assert hashlib.sha256(a.tobytes()).hexdigest() == d["sha256_A"]
    assert hashlib.sha256(wp.tobytes()).hexdigest() == d["sha256_Wp"]
    # the reference's own benchmark shapes also through the drop-ins of its two CUDA entry points
    paths = ("auto", "gemm", "tiled", "naive") if name.startswith("refbench") and case.M <= 2048 else ("auto", "gemm")
    for path in paths:
        log(f"[{path}] {name} M={case.M} K={case.K} N={case.N}")
        got = run(path, a, wp, case.N)
        assert [int(x) for x in got.ravel()[:8]] == d["C_first8"], (path, name)
        assert int(got.astype(np.int64).sum()) == d["C_checksum_int64"], (path, name)
        assert hashlib.sha256(got.tobytes()).hexdigest() == d["sha256_C"], (path, name)
        if name == "cfg5_worst":
            assert (got == 2097152).all()
        del got


@pytest.mark.parametrize("capture", [False, True])
def test_split_k_repeated_launches_exact(oracle, capture):
    """Split-K partial sums go through the workspace and either a reduce launch or, for few splits of
    the wave GEMV, the last-arriving workgroup of each strip (arrival counters that every call leaves
    at zero); every one of many back-to-back launches must be bit-exact.  capture=True records the launches into a hipGraph on
    a fresh stream (no workspace can be allocated while capturing, so the split-K falls back to
    zero-fill + atomics) and replays it several times, checking each replay."""
    s = hr.Stream()
    if capture:
        for name in ("cfg2_up", "cfg3_m4_up"):
            case = configs.CASES[name]
            a, wp = configs.gen_a(case), configs.gen_w_packed(case)
            expect = oracle.mm("scalar_mt", a, wp, case.N)
            da, db = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp)
            dc = hr.DeviceBuffer(4 * case.M * case.N)
            log(f"[graph] {name}")
            g = hr.Graph(s, lambda: [tx.mul_mat_ternary(da.value, db.value, dc.value, case.M, case.K, case.N,
                                                        stream=s.handle) for _ in range(3)])
            for rep in range(5):
                dc.upload(np.full(case.M * case.N, GARBAGE, np.int32))
                g.launch()
                s.synchronize()
                assert (dc.download(np.int32, (case.M, case.N)) == expect).all(), (name, rep)
        return
    for name in ("cfg2_up", "cfg2_down", "cfg3_m4_up", "cfg3_m16_down"):
        case = configs.CASES[name]
        a, wp = configs.gen_a(case), configs.gen_w_packed(case)
        expect = oracle.mm("scalar_mt", a, wp, case.N)
        da, db = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp)
        dc = hr.DeviceBuffer(4 * case.M * case.N)
        log(f"[eager] {name}: 120 launches")
        for it in range(120):
            dc.upload(np.full(case.M * case.N, GARBAGE, np.int32))
            st = tx.mul_mat_ternary(da.value, db.value, dc.value, case.M, case.K, case.N, stream=s.handle)
            assert st == 0
            s.synchronize()
            got = dc.download(np.int32, (case.M, case.N))
            assert (got == expect).all(), (name, it)
        # back-to-back without host sync in between, then check the final one
        for it in range(200):
            assert tx.mul_mat_ternary(da.value, db.value, dc.value, case.M, case.K, case.N, stream=s.handle) == 0
        s.synchronize()
        assert (dc.download(np.int32, (case.M, case.N)) == expect).all(), name


def test_single_launch_split_k_interleaved_and_graph(oracle):
    """The wave GEMV's in-launch split-K sum (cfg1, cfg2 up, cfg3 M=4 up, 24 rows in two m-groups,
    tile-64 weights) shares one set of arrival counters per stream: calls of different shapes issued
    back to back without host synchronisation, and a graph of them captured after the counters exist
    and replayed with eager calls between replays, all give the oracle's C."""
    s = hr.Stream()
    rng = np.random.default_rng(33)
    probs = []
    for m, k, n, tiled in ((1, 2560, 2560, 0), (1, 2560, 6912, 0), (4, 4096, 11008, 0), (24, 2048, 4096, 0),
                           (2, 4096, 4096, 1), (1, 2560, 6912, 1)):
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        expect = oracle.mm("scalar_mt", a, wp, n)
        w_dev = tx.interleave_tile64(wp) if tiled else wp
        da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(w_dev), hr.DeviceBuffer(4 * m * n)
        probs.append((m, k, n, "tile64" if tiled else "auto", da, db, dc, expect))

    def issue_all():
        for m, k, n, path, da, db, dc, _ in probs:
            assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n, stream=s.handle, path=path) == 0

    def check(tag):
        for m, k, n, path, _, _, dc, expect in probs:
            assert (dc.download(np.int32, (m, n)) == expect).all(), (tag, m, k, n, path)

    log("[in-launch split-K] interleaved eager calls")
    for it in range(40):
        issue_all()
    s.synchronize()
    check("eager")
    log("[in-launch split-K] graph replays")
    g = hr.Graph(s, issue_all)
    for rep in range(4):
        for _, _, _, _, _, _, dc, _ in probs:
            dc.upload(np.full(dc.nbytes // 4, GARBAGE, np.int32))
        g.launch()
        s.synchronize()
        check(f"replay {rep}")
        issue_all()  # eager work between replays
        s.synchronize()
        check(f"eager after replay {rep}")


def test_single_launch_split_k_two_streams(oracle):
    """Two streams run the in-launch split-K sum concurrently (each stream has its own counters and
    partials): alternating calls without synchronisation give the oracle's C on both."""
    s1, s2 = hr.Stream(), hr.Stream()
    rng = np.random.default_rng(34)
    jobs = []
    for s, (m, k, n) in ((s1, (1, 2560, 6912)), (s2, (1, 2560, 6912)), (s1, (4, 4096, 4096)), (s2, (3, 6912, 2560))):
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n)
        jobs.append((s, m, k, n, da, db, dc, oracle.mm("scalar_mt", a, wp, n)))
    log("[in-launch split-K] two streams")
    for it in range(50):
        for s, m, k, n, da, db, dc, _ in jobs:
            assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n, stream=s.handle) == 0
    s1.synchronize()
    s2.synchronize()
    for _, m, k, n, _, _, dc, expect in jobs:
        assert (dc.download(np.int32, (m, n)) == expect).all(), (m, k, n)


def test_host_threads_on_own_streams(oracle):
    """Four host threads (ctypes releases the GIL) each drive their own stream: the per-(device,
    stream) workspace, arrival counters and the device-property cache are created concurrently, and
    every result is exact."""
    import threading
    rng = np.random.default_rng(35)
    shapes = ((1, 2560, 6912), (4, 4096, 4096), (16, 11008, 4096), (64, 4096, 2048), (1, 6912, 2560))
    cases = []
    for m, k, n in shapes:
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        cases.append((m, k, n, hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp),
                      oracle.mm("scalar_mt", a, wp, n)))
    errors = []

    def worker(t):
        try:
            s = hr.Stream()
            outs = [hr.DeviceBuffer(4 * m * n) for m, k, n, *_ in cases]
            for it in range(20):
                for (m, k, n, da, db, _), dc in zip(cases, outs):
                    st = tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n, stream=s.handle)
                    if st != 0:
                        errors.append((t, it, m, k, n, st))
                        return
            s.synchronize()
            for (m, k, n, _, _, expect), dc in zip(cases, outs):
                if not (dc.download(np.int32, (m, n)) == expect).all():
                    errors.append((t, "mismatch", m, k, n))
        except Exception as e:  # reported below
            errors.append((t, repr(e)))

    log("[threads] 4 host threads, own streams")
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors


def test_random_shapes_all_planners(oracle):
    """Seeded random shapes across every planner branch (wave GEMV with and without in-launch split
    sums, DMA-staged GEMV, padded ragged path, narrow and wide GEMMs with and without split-K), on the
    automatic path and, where the shape allows, on tile-64 weights; each compared with the oracle."""
    rng = np.random.default_rng(2024)
    s = hr.Stream()
    done = 0
    for t in range(40):
        m = int(rng.choice([1, 2, 3, 4, 5, 8, 16, 17, 24, 32, 33, 48, 64, 65, 96, 128, 200]))
        k = int(rng.integers(1, 9000)) if t % 2 else int(rng.integers(1, 70)) * 128
        n = 4 * int(rng.integers(1, 3000)) if t % 3 else 256 * int(rng.integers(1, 40))
        if m * k * n > 5e8:
            continue
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        wp &= 0xFF ^ ((wp & 0xAA) & ~((wp & 0x55) << 1) & 0xAA)  # no code 10
        expect = oracle.mm("scalar_mt", a, wp, n)
        log(f"[random] M={m} K={k} N={n}")
        da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n)
        dc.upload(np.full(m * n, GARBAGE, np.int32))
        assert tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n, stream=s.handle) == 0
        s.synchronize()
        assert (dc.download(np.int32, (m, n)) == expect).all(), ("auto", m, k, n)
        if k % 128 == 0 and n % 256 == 0:
            dt = hr.DeviceBuffer(wp.nbytes)
            assert tx.interleave_tile64_device(dt.value, db.value, k, n, s.handle) == 0
            dc.upload(np.full(m * n, GARBAGE, np.int32))
            assert tx.mul_mat_ternary(da.value, dt.value, dc.value, m, k, n, stream=s.handle, path="tile64") == 0
            s.synchronize()
            assert (dc.download(np.int32, (m, n)) == expect).all(), ("tile64", m, k, n)
        done += 1
    assert done >= 20


def test_graph_survives_workspace_growth(oracle):
    """A graph captured while the stream's split-K workspace is small keeps working after a larger
    shape on the same stream grows the workspace (outgrown buffers are retired, never freed)."""
    s = hr.Stream()
    small = configs.CASES["cfg1"]
    a, wp = configs.gen_a(small), configs.gen_w_packed(small)
    expect = oracle.mm("scalar_mt", a, wp, small.N)
    da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * small.N)
    assert tx.mul_mat_ternary(da.value, db.value, dc.value, small.M, small.K, small.N, stream=s.handle) == 0
    s.synchronize()  # workspace now allocated for this stream: the graph below records the split-K path
    log("[graph + growth] capture cfg1")
    g = hr.Graph(s, lambda: tx.mul_mat_ternary(da.value, db.value, dc.value, small.M, small.K, small.N,
                                               stream=s.handle))
    # M=16, K=1 << 16, N=16384: 16 splits x 16 x 16384 int32 partials = 16 MiB > the first 8 MiB workspace
    m, k, n = 16, 1 << 16, 16384
    rng = np.random.default_rng(4)
    a2 = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    w2 = tx.pack_ternary((rng.integers(0, 3, size=(k, n)) - 1).astype(np.int8))
    d2a, d2b, d2c = hr.DeviceBuffer.from_array(a2), hr.DeviceBuffer.from_array(w2), hr.DeviceBuffer(4 * m * n)
    log("[graph + growth] large eager call")
    assert tx.mul_mat_ternary(d2a.value, d2b.value, d2c.value, m, k, n, stream=s.handle) == 0
    s.synchronize()
    for rep in range(3):
        dc.upload(np.full(small.N, GARBAGE, np.int32))
        g.launch()
        s.synchronize()
        assert (dc.download(np.int32, (1, small.N)) == expect).all(), rep
    got = d2c.download(np.int32, (m, n))
    assert (got[:2] == oracle.mm("scalar", a2[:2], w2, n)).all()


def test_padded_path_graph_replay(oracle):
    """Ragged and misaligned shapes on the automatic path (padded copy in the stream's workspace, aligned
    kernels, padding-dropping reduce) captured into a hipGraph after one eager call has sized the
    workspace; every replay, with eager work on the stream between replays, gives the oracle's C."""
    s = hr.Stream()
    rng = np.random.default_rng(21)
    shapes = ((1, 1000, 3076, 0), (17, 4093, 1028, 0), (129, 1001, 516, 0), (3, 4096, 1024, 3), (40, 512, 256, 1))
    for m, k, n, off in shapes:
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        wp &= 0xFF ^ ((wp & 0xAA) & ~((wp & 0x55) << 1) & 0xAA)  # clear code 10 fields (10 -> 00)
        expect = oracle.mm("scalar", a, wp, n)
        da, db, dc = hr.DeviceBuffer(a.nbytes + 16), hr.DeviceBuffer(wp.nbytes + 16), hr.DeviceBuffer(4 * m * n)
        hr.check(hr._load().hipMemcpy(ctypes.c_void_p(da.value + off), a.ctypes.data_as(ctypes.c_void_p), a.nbytes,
                                      hr.H2D), "A")
        hr.check(hr._load().hipMemcpy(ctypes.c_void_p(db.value + off), wp.ctypes.data_as(ctypes.c_void_p),
                                      wp.nbytes, hr.H2D), "W")
        call = lambda: tx.mul_mat_ternary(da.value + off, db.value + off, dc.value, m, k, n, stream=s.handle)
        log(f"[padded graph] M={m} K={k} N={n} offset={off}")
        assert call() == 0
        s.synchronize()
        assert (dc.download(np.int32, (m, n)) == expect).all(), "eager"
        g = hr.Graph(s, call)
        for rep in range(3):
            dc.upload(np.full(m * n, GARBAGE, np.int32))
            g.launch()
            s.synchronize()
            assert (dc.download(np.int32, (m, n)) == expect).all(), (m, k, n, rep)
            assert call() == 0  # eager work between replays
            s.synchronize()


@pytest.mark.parametrize("m,k,n", [(1, 64, 1024), (1, 2560, 1024), (3, 4032, 2048), (4, 4096, 512), (8, 1024, 4096),
                                   (16, 4096, 1024), (17, 2048, 1024), (24, 4096, 512), (32, 2560, 1024),
                                   (12, 8192, 512), (20, 6144, 1024), (2, 8192, 256)])
def test_wave_kernel_shapes(oracle, m, k, n):
    """Shapes the wave-pipelined skinny kernel takes on the automatic path: one launch for K <= 4096
    (1, 2 or 3 m-groups, 1-row and 4-row groups, one k-step), a few K splits for 4 < M with longer K;
    and M <= 4 with long K, which stays on the DMA-staged kernel."""
    rng = np.random.default_rng(m * 7 + k)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    log(f"[wave] M={m} K={k} N={n}")
    assert (run("auto", a, wp, n) == oracle.mm("scalar_mt", a, wp, n)).all()


@pytest.mark.parametrize("m,k,n,splits", [(17, 4096, 4096, 6), (24, 2560, 6912, 5), (32, 6912, 2560, 6),
                                          (40, 4096, 4096, 5), (48, 4096, 4096, 5), (64, 6912, 2560, 6)])
def test_several_m_groups_self_zeroing_wave(oracle, m, k, n, splits):
    """Aligned operands with 17-64 rows take the wave-pipelined kernel's self-zeroing plan, about two
    workgroups per CU (not the ragged form of the whole-line GEMV, whose two row groups are for ragged
    operands), bit-exact against the oracle on two calls in a row."""
    lib = tx._load()
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, m, k, n, buf, len(buf)) == 0
    plan = buf.value.decode()
    assert plan.startswith("skinny_wave_kernel sw=32"), plan
    if hr.device_attribute(hr.ATTR_MULTIPROCESSOR_COUNT) == 256:
        assert f"splits={splits} " in plan, plan
    rng = np.random.default_rng(m * 31 + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    expect = oracle.mm("scalar_mt", a, wp, n)
    log(f"[wave m-groups] M={m} K={k} N={n} {plan[:44]}")
    for rep in range(2):
        assert (run("auto", a, wp, n) == expect).all(), rep


@pytest.mark.parametrize("m,k,n,rows,splits", [(96, 8192, 2048, 64, 16), (128, 6144, 8192, 64, 4),
                                               (256, 8192, 2048, 64, 8), (512, 11008, 4096, 128, 4),
                                               (384, 11008, 4096, 128, 5)])
def test_split_gemm_tile_height(oracle, m, k, n, rows, splits):
    """Split-K GEMMs: 64-row or 128-row tiles with the split count sized to one workgroup per CU, the
    128-row ones where they keep more CUs busy or carry >= 80 M multiply-adds per workgroup (plans on
    a 256-CU device), bit-exact against the oracle on two calls in a row."""
    lib = tx._load()
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, m, k, n, buf, len(buf)) == 0
    plan = buf.value.decode()
    if hr.device_attribute(hr.ATTR_MULTIPROCESSOR_COUNT) == 256:
        assert plan.startswith(f"gemm_pipe_kernel<{rows} rows x 256 cols"), plan
        assert f"splits={splits} " in plan, plan
    rng = np.random.default_rng(m + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    expect = oracle.mm("scalar_mt", a, wp, n)
    log(f"[split GEMM tiles] M={m} K={k} N={n} {plan[:60]}")
    for rep in range(2):
        assert (run("auto", a, wp, n) == expect).all(), rep


@pytest.mark.parametrize("m,k,n,kernel", [(48, 2560, 6912, "gemm_pipe_kernel<64 rows x 64 cols"),
                                          (64, 2048, 8192, "gemm_pipe_kernel<64 rows x 64 cols"),
                                          (48, 4096, 4096, "skinny_wave_kernel"),
                                          (64, 6912, 2560, "skinny_wave_kernel")])
def test_many_rows_wave_or_narrow_gemm(oracle, m, k, n, kernel):
    """33-64 rows: the unsplit narrow GEMM where it has at least 96 column tiles, else the
    wave-pipelined kernel's split plan (plans on a 256-CU device), bit-exact against the oracle."""
    lib = tx._load()
    buf = ctypes.create_string_buffer(192)
    assert lib.ternix_hip_plan_describe(1 << 20, 1 << 24, m, k, n, buf, len(buf)) == 0
    plan = buf.value.decode()
    if hr.device_attribute(hr.ATTR_MULTIPROCESSOR_COUNT) == 256:
        assert plan.startswith(kernel), plan
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
    expect = oracle.mm("scalar_mt", a, wp, n)
    log(f"[rows 33-64] M={m} K={k} N={n} {plan[:50]}")
    assert (run("auto", a, wp, n) == expect).all()
