"""Device-side weight format (ternix_hip_pack/unpack/interleave_weights_offline) against the CPU oracle
(oracle/ternix_oracle.c, a restatement of reference src/bitpack.cpp:5-33), byte for byte.

Inputs cover every int8 value (only +1 and -1 have codes; all others pack to 00, as in the
reference), every 2-bit code on the way back (10 unpacks to 0), sizes that are not multiples of 4,
16 or 64 (the trailing size % 4 weights are ignored, bytes past size/4 are never written), and
misaligned buffers (byte path)."""
import ctypes
import hashlib
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import ternixengine_amd as tx  # noqa: E402
from ternixengine_amd import configs  # noqa: E402
from ternixengine_amd import hip_runtime as hr  # noqa: E402

SENTINEL = 0xA5


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if hr.device_count() < 1:
        pytest.skip("no HIP device")
    tx._load()
    yield


def oracle_pack(oracle, w):
    out = np.full(w.size // 4, SENTINEL, np.uint8)
    oracle.lib.oracle_pack_ternary(out.ctypes.data_as(ctypes.c_void_p), w.ctypes.data_as(ctypes.c_void_p), w.size)
    return out


def oracle_unpack(oracle, p, size):
    out = np.full(size, SENTINEL, np.uint8).view(np.int8)
    oracle.lib.oracle_unpack_ternary(out.ctypes.data_as(ctypes.c_void_p), p.ctypes.data_as(ctypes.c_void_p), size)
    return out


def device_pack(w, off_in=0, off_out=0):
    size = w.size
    din = hr.DeviceBuffer(size + off_in + 16)
    dout = hr.DeviceBuffer(size // 4 + off_out + 16)
    dout.upload(np.full(size // 4 + off_out + 16, SENTINEL, np.uint8))
    if size:
        hr.check(hr._load().hipMemcpy(din.value + off_in, w.ctypes.data, size, hr.H2D), "upload")
    st = tx.pack_ternary_device(dout.value + off_out, din.value + off_in, size)
    assert st == 0, tx.ternix_error(st)
    hr.synchronize()
    got = dout.download(np.uint8, (size // 4 + off_out + 16,))
    return got[off_out:off_out + size // 4], got[off_out + size // 4:]


def device_unpack(p, size, off_in=0, off_out=0):
    din = hr.DeviceBuffer(p.size + off_in + 16)
    dout = hr.DeviceBuffer(size + off_out + 16)
    dout.upload(np.full(size + off_out + 16, SENTINEL, np.uint8))
    if p.size:
        hr.check(hr._load().hipMemcpy(din.value + off_in, p.ctypes.data, p.size, hr.H2D), "upload")
    st = tx.unpack_ternary_device(dout.value + off_out, din.value + off_in, size)
    assert st == 0, tx.ternix_error(st)
    hr.synchronize()
    got = dout.download(np.uint8, (size + off_out + 16,))
    n = 4 * (size // 4)
    return got[off_out:off_out + n].view(np.int8), got[off_out + n:]


SIZES = [0, 3, 4, 7, 64, 68, 1000, 4096, 4099, 65536 + 12, 1 << 20]


@pytest.mark.parametrize("size", SIZES)
def test_pack_matches_oracle_all_int8_values(oracle, size):
    log(f"[pack] size={size}")
    rng = np.random.default_rng(size)
    w = rng.integers(-128, 128, size=size, dtype=np.int16).astype(np.int8)
    # make +-1 common so every code appears
    mask = rng.random(size)
    w[mask < 0.3] = 1
    w[(mask >= 0.3) & (mask < 0.6)] = -1
    got, tail = device_pack(w)
    np.testing.assert_array_equal(got, oracle_pack(oracle, w))
    assert (tail == SENTINEL).all(), "bytes past size/4 were written"


@pytest.mark.parametrize("size", SIZES)
def test_unpack_matches_oracle_all_codes(oracle, size):
    log(f"[unpack] size={size}")
    rng = np.random.default_rng(size + 1)
    p = rng.integers(0, 256, size=size // 4, dtype=np.int16).astype(np.uint8)  # includes code 10
    got, tail = device_unpack(p, size)
    np.testing.assert_array_equal(got, oracle_unpack(oracle, p, size)[:4 * (size // 4)])
    assert (tail == SENTINEL).all(), "elements past 4*(size/4) were written"


@pytest.mark.parametrize("offs", [(1, 0), (0, 3), (5, 7)])
def test_misaligned_buffers(oracle, offs):
    log(f"[pack/unpack misaligned] offsets={offs}")
    rng = np.random.default_rng(7)
    w = (rng.integers(0, 3, size=5000) - 1).astype(np.int8)
    got, tail = device_pack(w, *offs)
    np.testing.assert_array_equal(got, oracle_pack(oracle, w))
    assert (tail == SENTINEL).all()
    back, tail = device_unpack(got, w.size, *offs)
    np.testing.assert_array_equal(back, w[:4 * (w.size // 4)])
    assert (tail == SENTINEL).all()


def test_round_trip_and_known_answer():
    log("[pack] known answer")
    w = np.array([1, 0, -1, 1, -1, 0, 1, 0], np.int8)  # reference tests/test_bitpack.cpp:6
    got, _ = device_pack(w)
    assert got.tolist() == [0x71, 0x13]
    back, _ = device_unpack(got, 8)
    np.testing.assert_array_equal(back, w)


def test_full_size_weights_match_committed_digest(digests):
    """Pack the cfg5 big weights (K=8192, N=28672, 58.7 MB packed) on the GPU from the unpacked
    synthetic matrix; the bytes must hash to the digest the reference's own packer produced."""
    case = configs.CASES["cfg5_big_m1"]
    log(f"[pack] full size {case.K}x{case.N}")
    w = configs.gen_w(case)
    got, _ = device_pack(w.reshape(-1))
    assert hashlib.sha256(got.tobytes()).hexdigest() == digests[case.name]["sha256_Wp"]


def test_interleave_is_device_copy():
    log("[interleave]")
    rng = np.random.default_rng(3)
    p = rng.integers(0, 256, size=1024, dtype=np.int16).astype(np.uint8)
    din, dout = hr.DeviceBuffer.from_array(p), hr.DeviceBuffer(1024)
    assert tx._load().ternix_hip_interleave_weights_offline(dout.value, din.value, 4096, None) == 0
    hr.synchronize()
    np.testing.assert_array_equal(dout.download(np.uint8, (1024,)), p)
