"""Asynchronous results are never touched before their wait, in the gfx950 assembly built here.

Several kernels issue LDS reads (ds_read_b64_tr_b8, ds_read_b128) and returning atomics or loads
(global_atomic_add_x2 ... sc0, global_load ... sc1) as inline assembly, so that the compiler does
not place its own waits; the compiler then treats their destination registers as written at issue.
Correctness rests on every later instruction that reads, moves or overwrites those registers coming
after an s_waitcnt that covers the operation.  This test checks exactly that, for every instruction
that writes vector registers asynchronously (inline assembly or not), in every kernel of every .hip
file of the library: walking forward in program order from the operation, the first instruction
that names any of its destination registers must come after a wait whose count (lgkmcnt for LDS,
vmcnt for global memory) is at most the number of operations of the same kind issued after it
(0 when other kinds are mixed in: LDS with scalar loads, loads with stores).  A later plain load that
only overwrites those registers ends the walk: loads return in issue order, so its data lands last (the
compiler lays out both halves of an exec-masked if / else in sequence, each loading into the same
registers for its own lanes).  The walk follows the fall-through path and stops at an unconditional
jump or the end of the program."""
import os
import re
import subprocess

import pytest

from conftest import hip_file_flags

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ternixengine_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
SOURCES = ["skinny_kernels.hip", "line_gemv.hip", "gemm_kernels.hip", "skinny_deep.hip", "layer_kernels.hip",
           "ffn_kernels.hip", "bitpack_kernels.hip"]

_VREG = re.compile(r"\bv(?:(\d+)|\[(\d+):(\d+)\])")


def _vregs(text):
    out = set()
    for m in _VREG.finditer(text):
        if m.group(1) is not None:
            out.add(int(m.group(1)))
        else:
            out.update(range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def _parse(line):
    """(mnemonic, operand text) of an instruction line, or None for labels, directives, comments."""
    s = line.split(";", 1)[0].strip()
    if not s or s.startswith(".") or s.endswith(":"):
        return None
    parts = s.split(None, 1)
    return parts[0], (parts[1] if len(parts) > 1 else "")


def _async_dest(mn, ops):
    """('lgkm' | 'vm', destination registers) for an instruction that writes VGPRs asynchronously."""
    if mn.startswith("ds_read") or (mn.startswith("ds_") and "rtn" in mn):
        return "lgkm", _vregs(ops.split(",", 1)[0])
    if mn.startswith(("global_load", "buffer_load", "scratch_load")) and "lds" not in mn:
        if mn.startswith("buffer_load") and " lds" in ops:
            return None
        return "vm", _vregs(ops.split(",", 1)[0])
    if mn.startswith(("global_atomic", "buffer_atomic")) and re.search(r"\bsc0\b", ops):
        return "vm", _vregs(ops.split(",", 1)[0])
    return None


def _plain_load(mn):
    """A load from global memory into VGPRs (not an atomic, not LDS-bound): such loads return their
    data in issue order on vmcnt."""
    return mn.startswith(("global_load", "buffer_load")) and "lds" not in mn


def _kind(mn):
    if mn.startswith("ds_"):
        return "lgkm"
    if mn.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_dcache")):
        return "smem"
    if mn.startswith(("global_", "buffer_", "scratch_")):
        return "vm_store" if ("store" in mn or ("atomic" in mn and "sc0" not in mn)) else "vm"
    return None


def _waits(ops):
    w = {}
    for name, key in (("vmcnt", "vm"), ("lgkmcnt", "lgkm")):
        m = re.search(name + r"\((\d+)\)", ops)
        if m:
            w[key] = int(m.group(1))
    return w


def hazards(lines):
    insts = [p for p in (_parse(l) for l in lines) if p is not None]
    found = []
    for i, (mn, ops) in enumerate(insts):
        a = _async_dest(mn, ops)
        if not a or not a[1]:
            continue
        kind, dest = a
        same = other = 0  # operations of the same counter issued after i; of another kind sharing it
        for j in range(i + 1, len(insts)):
            mj, oj = insts[j]
            if mj == "s_waitcnt":
                w = _waits(oj)
                if kind in w and w[kind] <= (same if other == 0 else 0):
                    break  # operation i has completed
                continue
            if _vregs(oj) & dest:
                if _plain_load(mn) and _plain_load(mj) and not (_vregs(oj.split(",", 1)[1]) & dest):
                    break  # a later load only overwrites them: loads return in order, so it lands last
                found.append(f"{mn} {ops}  ->  {mj} {oj}")
                break
            k = _kind(mj)
            if kind == "lgkm":
                same += k == "lgkm"
                other += k == "smem"
            else:
                same += k == "vm"
                other += k == "vm_store"
            if mj in ("s_branch", "s_setpc_b64", "s_endpgm"):
                break
    return found


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("isa_async")
    funcs = {}
    for src in SOURCES:
        out = d / (src + ".s")
        subprocess.run([HIPCC, "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        "-O3", "-std=c++17", f"-I{ROOT}/include", f"-I{CSRC}", "--cuda-device-only", "-S", "-o",
                        str(out), os.path.join(CSRC, src)] + hip_file_flags(src), check=True, capture_output=True,
                       timeout=900)
        text = out.read_text()
        for m in re.finditer(r"^(_Z\w*):\s*(?:;.*)?$", text, re.M):
            end = text.find(".Lfunc_end", m.end())
            if end > 0:
                funcs[(src, m.group(1))] = text[m.end():end].splitlines()
    return funcs


def test_checker_finds_a_planted_hazard():
    bad = ["ds_read_b64_tr_b8 v[20:21], v4", "v_mov_b32_e32 v30, v20", "s_waitcnt lgkmcnt(0)"]
    good = ["ds_read_b64_tr_b8 v[20:21], v4", "ds_read_b64_tr_b8 v[22:23], v5", "s_waitcnt lgkmcnt(1)",
            "v_mov_b32_e32 v30, v20"]
    early = ["ds_read_b64_tr_b8 v[20:21], v4", "ds_read_b64_tr_b8 v[22:23], v5", "s_waitcnt lgkmcnt(1)",
             "v_mov_b32_e32 v30, v22"]
    atomic = ["global_atomic_add_x2 v[6:7], v[2:3], v[0:1], off sc0", "v_readfirstlane_b32 s9, v7",
              "s_waitcnt vmcnt(0)"]
    overwrite = ["global_load_dwordx2 v[8:9], v[4:5], off sc1", "v_mov_b32_e32 v8, 0", "s_waitcnt vmcnt(0)"]
    # two exec-masked loads into the same registers (an if / else the compiler laid out in sequence):
    # ordered by the in-order return of loads; a later load that addresses with them reads them early
    waw = ["global_load_dwordx4 v[6:9], v[20:21], off", "global_load_dword v6, v[22:23], off",
           "s_waitcnt vmcnt(0)", "v_mov_b32_e32 v30, v6"]
    addr = ["global_load_dwordx2 v[6:7], v[20:21], off", "global_load_dword v8, v[6:7], off", "s_waitcnt vmcnt(0)"]
    assert hazards(bad) and hazards(early) and hazards(atomic) and hazards(overwrite) and hazards(addr)
    assert not hazards(good) and not hazards(waw)


def test_no_async_register_hazards(kernels):
    names = [k for k in kernels if "line_gemv_kernel" in k[1] or "gemm_pipe_kernel" in k[1] or
             "skinny_wave_kernel" in k[1]]
    assert names, "expected kernels not found in the assembly"
    bad = {}
    for key, lines in kernels.items():
        h = hazards(lines)
        if h:
            bad[f"{key[0]}:{key[1]}"] = h[:3]
    assert not bad, bad
