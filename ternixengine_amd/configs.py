"""The benchmark configurations this path is measured and checked on, with their synthetic inputs.

Each case is one (M, K, N) product with a fixed input distribution.  Inputs come from the library's
deterministic generators (include/ternix/synth.h) with seed 0 and a per-case stream id, so every
platform gets identical bytes (the reference's std::mt19937 streams are not portable).
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import load as _load

Q32 = 1 << 32


@dataclass(frozen=True)
class Case:
    name: str
    config: int
    M: int
    K: int
    N: int
    act: str          # "uniform" | "gauss32" | "const-128"
    p_neg: float      # P(w = -1)
    p_pos: float      # P(w = +1)
    stream: int       # A uses stream 2*stream, W uses 2*stream+1

    @property
    def bytes_algorithmic(self):
        """Each operand once: M*K (A) + K*N/4 (packed W) + 4*M*N (C)."""
        return self.M * self.K + self.K * self.N // 4 + 4 * self.M * self.N

    @property
    def ops(self):
        return 2 * self.M * self.N * self.K


def _cases():
    out = []
    sid = 0

    def add(name, cfg, m, k, n, act, pn, pp):
        nonlocal sid
        out.append(Case(name, cfg, m, k, n, act, pn, pp, sid))
        sid += 1

    add("cfg1", 1, 1, 2560, 2560, "uniform", 0.3, 0.3)
    add("cfg2_up", 2, 1, 2560, 6912, "uniform", 0.3, 0.3)
    add("cfg2_down", 2, 1, 6912, 2560, "uniform", 0.3, 0.3)
    for m in (4, 16, 64):
        add(f"cfg3_m{m}_up", 3, m, 4096, 11008, "gauss32", 0.25, 0.25)
        add(f"cfg3_m{m}_down", 3, m, 11008, 4096, "gauss32", 0.25, 0.25)
    for k, n in ((4096, 4096), (4096, 14336), (14336, 4096)):
        add(f"cfg4_{k}x{n}", 4, 2048, k, n, "uniform", 0.325, 0.325)
    third = 1.0 / 3.0
    for m, k, n in ((1, 1000, 3076), (17, 4093, 1028), (129, 8191, 2052)):
        add(f"cfg5_ragged_{m}x{k}x{n}", 5, m, k, n, "uniform", third, third)
    add("cfg5_big_m1", 5, 1, 8192, 28672, "uniform", third, third)
    add("cfg5_big_m4096", 5, 4096, 8192, 28672, "uniform", third, third)
    add("cfg5_worst", 5, 256, 16384, 4096, "const-128", 1.0, 0.0)
    # The reference's own GPU benchmark (benchmarks/bench_cuda.cu:45-50): square n^3 problems, A uniform
    # int8, W uniform over {-1, 0, +1}; its published figures are for these shapes (README.md:178-181).
    for n in (512, 1024, 2048, 4096):
        add(f"refbench_n{n}", 0, n, n, n, "uniform", third, third)
    return out


CASES = {c.name: c for c in _cases()}


def _q(p):
    return min(int(round(p * Q32)), Q32)


def gen_a(case, seed=0):
    lib = _load()
    a = np.empty((case.M, case.K), dtype=np.int8)
    if case.act == "uniform":
        lib.ternix_synth_act_uniform(a.ctypes.data_as(ctypes.c_void_p), a.size, seed, 2 * case.stream)
    elif case.act == "gauss32":
        lib.ternix_synth_act_gauss(a.ctypes.data_as(ctypes.c_void_p), a.size, seed, 2 * case.stream, 32)
    elif case.act == "const-128":
        a.fill(-128)
    else:
        raise ValueError(case.act)
    return a


def gen_w_packed(case, seed=0):
    lib = _load()
    wp = np.empty((case.K, case.N // 4), dtype=np.uint8)
    lib.ternix_synth_ternary_packed(wp.ctypes.data_as(ctypes.c_void_p), case.K * case.N, seed,
                                    2 * case.stream + 1, _q(case.p_neg), _q(case.p_pos))
    return wp


def gen_w(case, seed=0):
    """Unpacked weights (K, N) int8 -- same values as gen_w_packed."""
    lib = _load()
    w = np.empty((case.K, case.N), dtype=np.int8)
    lib.ternix_synth_ternary(w.ctypes.data_as(ctypes.c_void_p), w.size, seed, 2 * case.stream + 1,
                             _q(case.p_neg), _q(case.p_pos))
    return w
