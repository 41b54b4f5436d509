"""Write the golden fixtures of this directory from the reference's own CPU code.

The reference kernels (src/mul_mat_ternary.cpp, src/bitpack.cpp) are compiled unchanged from
/root/reference by oracle/Makefile into oracle/_ref/libternix_ref.so; this script calls them through
ctypes on inputs from the library's deterministic generators (include/ternix/synth.h) and stores:

  small_cases.npz     inputs and reference outputs of the reference test-suite shapes
                      (tests/test_ternary_matmul.cpp:44, tests/test_cuda_matmul.cu:28-38,
                      tests/test_python_binding.py:28-31), plus the int8-extreme case
                      (tests/test_ternary_matmul.cpp:61-69) and an all-256-byte-values case that
                      exercises the out-of-domain code 10 in every reference kernel;
  config_digests.json SHA-256 of the A, packed-W and C bytes of every benchmark case
                      (ternixengine_amd/configs.py), C computed by the reference avx2_blocked kernel
                      (scalar where N % 8 != 0, the AVX2 precondition), multi-threaded over row blocks.

Run from the repository root:  python tests/golden/gen_golden.py [--skip-digests] [--only name,...]
"""
import argparse
import ctypes
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from ternixengine_amd import configs  # noqa: E402
from ternixengine_amd._lib import load as load_lib  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libternix_ref.so")


def load_ref():
    ref = ctypes.CDLL(REF_SO)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    for n in ("ref_mm_naive", "ref_mm_scalar", "ref_mm_avx2", "ref_mm_avx2_blocked"):
        getattr(ref, n).argtypes = [vp, vp, vp, sz, sz, sz]
    ref.ref_pack_ternary.argtypes = [vp, vp, sz]
    ref.ref_unpack_ternary.argtypes = [vp, vp, sz]
    ref.ref_mm_rows_mt.argtypes = [ctypes.c_int, vp, vp, vp, sz, sz, sz, ctypes.c_int]
    return ref


def p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def ref_mm(ref, name, a, wp, m, k, n):
    c = np.full((m, n), -999, dtype=np.int32)  # prefilled like the reference tests (:48)
    getattr(ref, name)(p(a), p(wp), p(c), m, k, n)
    return c


def small_cases(ref):
    lib = load_lib()
    shapes = [(1, 8, 8), (4, 16, 8), (5, 33, 24), (8, 64, 64), (13, 100, 40), (64, 256, 128),
              (64, 64, 64), (37, 100, 52), (128, 256, 192), (1, 32, 24)]
    out = {}
    for idx, (m, k, n) in enumerate(shapes):
        a = np.empty((m, k), np.int8)
        lib.ternix_synth_act_uniform(p(a), a.size, 7, 1000 + 2 * idx)
        w = np.empty((k, n), np.int8)
        third = int(round(2 ** 32 / 3))
        lib.ternix_synth_ternary(p(w), w.size, 7, 1001 + 2 * idx, third, third)
        wp = np.empty((k, n // 4), np.uint8)
        ref.ref_pack_ternary(p(wp), p(w), w.size)
        c = ref_mm(ref, "ref_mm_scalar", a, wp, m, k, n)
        # every reference kernel agrees on in-domain data; record that it was checked
        assert (ref_mm(ref, "ref_mm_naive", a, wp, m, k, n) == c).all()
        if n % 8 == 0:
            assert (ref_mm(ref, "ref_mm_avx2", a, wp, m, k, n) == c).all()
            assert (ref_mm(ref, "ref_mm_avx2_blocked", a, wp, m, k, n) == c).all()
        tag = f"s{idx}"
        out[f"{tag}_shape"] = np.array([m, k, n], np.int64)
        out[f"{tag}_A"] = a
        out[f"{tag}_W"] = w
        out[f"{tag}_Wp"] = wp
        out[f"{tag}_C"] = c
    out["n_small"] = np.array(len(shapes), np.int64)

    # Pack known answer (tests/test_bitpack.cpp:6).
    ka = np.array([1, 0, -1, 1, -1, 0, 1, 0], np.int8)
    kp = np.empty(2, np.uint8)
    ref.ref_pack_ternary(p(kp), p(ka), 8)
    out["pack_in"] = ka
    out["pack_out"] = kp

    # int8 extreme (tests/test_ternary_matmul.cpp:61-69): A == -128, random W, M=4, K=4096, N=16.
    m, k, n = 4, 4096, 16
    a = np.full((m, k), -128, np.int8)
    w = np.empty((k, n), np.int8)
    lib.ternix_synth_ternary(p(w), w.size, 7, 5001, int(round(2 ** 32 / 3)), int(round(2 ** 32 / 3)))
    wp = np.empty((k, n // 4), np.uint8)
    ref.ref_pack_ternary(p(wp), p(w), w.size)
    out["extreme_A"], out["extreme_Wp"] = a, wp
    out["extreme_C"] = ref_mm(ref, "ref_mm_avx2_blocked", a, wp, m, k, n)

    # Out-of-domain code 10: packed bytes take all 256 values; each reference kernel's own answer.
    m, k, n = 6, 256, 32
    a = np.empty((m, k), np.int8)
    lib.ternix_synth_act_uniform(p(a), a.size, 7, 6000)
    wp = np.empty((k, n // 4), np.uint8)
    wp.ravel()[:] = np.arange(wp.size) * 37 % 256
    out["invalid_A"], out["invalid_Wp"] = a, wp
    for name in ("naive", "scalar", "avx2", "avx2_blocked"):
        out[f"invalid_C_{name}"] = ref_mm(ref, f"ref_mm_{name}", a, wp, m, k, n)
    unp = np.empty((k, n), np.int8)
    ref.ref_unpack_ternary(p(unp), p(wp), unp.size)
    out["invalid_unpacked"] = unp
    return out


def sha(arr):
    return hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest()


def digests(ref, threads, only=None):
    res = {}
    for name, case in configs.CASES.items():
        if only and name not in only:
            continue
        t0 = time.time()
        a = configs.gen_a(case)
        wp = configs.gen_w_packed(case)
        c = np.full((case.M, case.N), -999, dtype=np.int32)
        impl = 2 if case.N % 8 == 0 else 0
        ref.ref_mm_rows_mt(impl, p(a), p(wp), p(c), case.M, case.K, case.N, threads)
        res[name] = {
            "M": case.M, "K": case.K, "N": case.N,
            "sha256_A": sha(a), "sha256_Wp": sha(wp), "sha256_C": sha(c),
            "reference_kernel": "mul_mat_ternary_avx2_blocked" if impl == 2 else "mul_mat_ternary_scalar",
            "C_checksum_int64": int(c.astype(np.int64).sum()),
            "C_first8": [int(x) for x in c.ravel()[:8]],
        }
        print(f"{name}: {time.time() - t0:.1f}s", flush=True)
        del a, wp, c
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-digests", action="store_true")
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--only", default="", help="comma-separated case names: (re)compute just these digests "
                                               "and keep the others already in config_digests.json")
    args = ap.parse_args()
    ref = load_ref()
    only = [x for x in args.only.split(",") if x]
    if not only:
        np.savez_compressed(os.path.join(HERE, "small_cases.npz"), **small_cases(ref))
    if not args.skip_digests:
        path = os.path.join(HERE, "config_digests.json")
        d = {}
        if only and os.path.exists(path):
            with open(path) as f:
                d = json.load(f)["cases"]
        d.update(digests(ref, args.threads, only))
        with open(path, "w") as f:
            json.dump({"generator": "ternixengine_amd.configs (seed 0)", "cases": d}, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
