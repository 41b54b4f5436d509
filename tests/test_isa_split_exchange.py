"""The in-launch split sum of the wave GEMV (skinny_kernels.hip, SK_LAST) exchanges partial sums
between workgroups with coherent accesses only: agent-scope relaxed atomic stores (global_store ...
sc1: written through to the device coherence point), a full vmcnt wait so they have completed
before the arrival counter's returning atomic, and agent-scope loads (global_load ... sc1) in the
last arriver, issued after the counter value came back.  That ordering is what makes the exchange
correct without the release/acquire cache maintenance (buffer_wbl2 / buffer_inv), and it rests on
the code the compiler emits, so this test reads the gfx950 assembly built here from the kernel
source and checks the sequence in every wave-kernel instantiation."""
import os
import re
import subprocess

import pytest

from conftest import hip_file_flags

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ternixengine_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def wave_kernels(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "skinny.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "-O3", "-std=c++17", f"-I{ROOT}/include", f"-I{CSRC}", "--cuda-device-only", "-S", "-o", str(out),
                    os.path.join(CSRC, "skinny_kernels.hip")] + hip_file_flags("skinny_kernels.hip"), check=True,
                   capture_output=True, timeout=600)
    text = out.read_text()
    funcs = {}
    for m in re.finditer(r"^(_Z\w*skinny_wave_kernel\w*):", text, re.M):
        end = text.find(".Lfunc_end", m.end())
        funcs[m.group(1)] = text[m.end():end].splitlines()
    return funcs


def _relaxed_exchange(lines):
    """Index of the relaxed arrival atomic (a returning 32-bit global_atomic_add not preceded by
    buffer_wbl2; the 64-bit ticket add of the self-zeroing mode is another exchange)."""
    for i, l in enumerate(lines):
        if re.search(r"global_atomic_add\s", l) and " sc0" in l and \
                not any("buffer_wbl2" in x for x in lines[max(0, i - 4):i]):
            return i
    return None


def test_wave_kernels_use_coherent_exchange(wave_kernels):
    # instantiations without fused quantisation take part in the in-launch split sum (the column-wave
    # form, last template argument true, only adds with atomics)
    names = [n for n in wave_kernels if re.search(r"skinny_wave_kernelILi(16|32)ELi\dELb[01]ELi0ELb0E", n)]
    assert names, "no wave-kernel instantiation found in the assembly"
    for name in names:
        lines = wave_kernels[name]
        i = _relaxed_exchange(lines)
        assert i is not None, name
        stores = [j for j in range(i) if re.search(r"global_store_dword\b.*\bsc1\b", lines[j])]
        assert stores, f"{name}: partial sums are not stored with sc1"
        between = lines[stores[-1] + 1:i]
        assert any(re.search(r"s_waitcnt vmcnt\(0\)", l) for l in between), \
            f"{name}: the arrival atomic is not preceded by a full vmcnt wait after the sc1 stores"
        # (sc1 loads before the atomic belong to the self-zeroing mode: its zeroed-word reads)
        loads = [j for j, l in enumerate(lines) if j > i and re.search(r"global_load_dwordx2\b.*\bsc1\b", l)]
        assert loads, f"{name}: last-arriver loads are not sc1 loads after the atomic"
        after = lines[i + 1:min(loads)]
        assert any(re.search(r"s_waitcnt vmcnt\(0\)", l) for l in after), \
            f"{name}: the last-arriver loads are issued before the counter value returned"


def test_self_zeroing_atomics_order(wave_kernels):
    """SK_ATOMZ (the M = 1 plan without a fill launch): the strip's first split zeroes its outputs
    with coherent stores (global_store_dwordx2 ... sc1), waits for every store (vmcnt(0)), and only
    then stores the zeroed word (sc1); the other splits read the zeroed word with a coherent load
    and wait for it before their first int32 atomic add into C."""
    names = [n for n in wave_kernels if re.search(r"skinny_wave_kernelILi(16|32)ELi\dELb1ELi0E", n)]
    assert names
    for name in names:
        lines = wave_kernels[name]
        ticket = [i for i, l in enumerate(lines) if "global_atomic_add_x2" in l and " sc0" in l]
        assert ticket, f"{name}: no returning 64-bit ticket add"
        t = ticket[0]
        zstores = [i for i, l in enumerate(lines) if i > t and re.search(r"global_store_dwordx2\b.*\bsc1\b", l)]
        assert len(zstores) >= 2, f"{name}: zero stores and zeroed-word store are not coherent 8-byte stores"
        flag = zstores[-1]
        zeros = zstores[:-1]
        between = lines[zeros[-1] + 1:flag]
        assert any(re.search(r"s_waitcnt vmcnt\(0\)", l) for l in between), \
            f"{name}: the zeroed word is stored before the zero stores completed"
        adds = [i for i, l in enumerate(lines) if re.search(r"global_atomic_add\b(?!_x2)", l) and " sc0" not in l]
        assert adds, f"{name}: no int32 atomic adds"
        zloads = [i for i, l in enumerate(lines) if re.search(r"global_load_dwordx2\b.*offset:8 sc1", l)]
        assert zloads and min(zloads) < min(adds), f"{name}: the zeroed word is not read before the atomics"
        assert any(re.search(r"s_waitcnt vmcnt\(0\)", l) for l in lines[min(zloads) + 1:min(adds)]), \
            f"{name}: the atomics may be issued before the zeroed word returned"
