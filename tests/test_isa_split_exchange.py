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
                    os.path.join(CSRC, "skinny_kernels.hip")], check=True, capture_output=True, timeout=600)
    text = out.read_text()
    funcs = {}
    for m in re.finditer(r"^(_Z\w*skinny_wave_kernel\w*):", text, re.M):
        end = text.find(".Lfunc_end", m.end())
        funcs[m.group(1)] = text[m.end():end].splitlines()
    return funcs


def _relaxed_exchange(lines):
    """Index of the relaxed arrival atomic (a returning global_atomic_add not preceded by buffer_wbl2)."""
    for i, l in enumerate(lines):
        if "global_atomic_add" in l and " sc0" in l and not any("buffer_wbl2" in x for x in lines[max(0, i - 4):i]):
            return i
    return None


def test_wave_kernels_use_coherent_exchange(wave_kernels):
    # instantiations without fused quantisation take part in the in-launch split sum
    names = [n for n in wave_kernels if re.search(r"skinny_wave_kernelILi(16|32)ELi\dELb[01]ELi0E", n)]
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
        loads = [j for j, l in enumerate(lines) if re.search(r"global_load_dwordx2\b.*\bsc1\b", l)]
        assert loads and min(loads) > i, f"{name}: last-arriver loads are not sc1 loads after the atomic"
        after = lines[i + 1:min(loads)]
        assert any(re.search(r"s_waitcnt vmcnt\(0\)", l) for l in after), \
            f"{name}: the last-arriver loads are issued before the counter value returned"
