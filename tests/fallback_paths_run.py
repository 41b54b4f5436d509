"""Child process of tests/test_fallback_paths.py: runs the automatic path on a fixed set of shapes
against the CPU oracle, with whatever TERNIX_* kernel switches the parent put in the environment
(the library reads them once, at first use), and exits non-zero on the first mismatch."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import ternixengine_amd as tx  # noqa: E402
from ternixengine_amd import hip_runtime as hr  # noqa: E402
from conftest import Oracle  # noqa: E402

SHAPES = [(1, 2560, 2560), (1, 6912, 2560), (4, 4096, 1024), (16, 2048, 4096), (16, 8192, 1024), (24, 4096, 512),
          (32, 2560, 1024), (48, 1024, 2048), (64, 4096, 1024), (129, 1001, 516), (1, 1000, 3076), (17, 4093, 1028),
          (256, 2048, 1024)]


def main():
    oracle = Oracle()
    rng = np.random.default_rng(5)
    for m, k, n in SHAPES:
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        wp = rng.integers(0, 256, size=(k, n // 4), dtype=np.uint8)
        da, db, dc = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wp), hr.DeviceBuffer(4 * m * n)
        dc.upload(np.full(m * n, -7, np.int32))
        print(f"M={m} K={k} N={n}", flush=True)
        st = tx.mul_mat_ternary(da.value, db.value, dc.value, m, k, n)
        if st != 0:
            print("status", st, tx.ternix_error(st))
            return 1
        hr.synchronize()
        if not (dc.download(np.int32, (m, n)) == oracle.mm("scalar_mt", a, wp, n)).all():
            print("MISMATCH")
            return 1
    print("all shapes bit-exact")
    return 0


if __name__ == "__main__":
    sys.exit(main())
