"""The wide GEMM tiles' asm-load ring, checked on the compiler's output.

gemm_wide_kernel (whetstone_amd/csrc/gemm.hip) issues its packed-weight loads
by inline asm into a ring of GW_DW = 4 register slots and waits for them with
hand-counted `s_waitcnt vmcnt`. The compiler takes an asm load's output
register as written when the load issues, so the scheme is only sound while
every ring slot keeps its physical registers from the prologue through every
loop round and the tail: a rename (a copy made while the load is still
landing) reads stale data. A 128-row variant of the kernel hit exactly that.

This test compiles gemm.hip for gfx950 with the build's own flags (hipcc, no
GPU needed) and reads, for every instantiation of the kernel, the destination
registers of its `global_load_dword` / `global_load_ubyte` in program order:
the RPT row-scale loads, then the prologue's four slots, then each loop round
and the tail must name the same registers slot for slot.
"""
import re
import shutil
import subprocess

import pytest

from whetstone_amd import build as B

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not
                                __import__("os").path.exists("/opt/rocm/bin/hipcc"),
                                reason="hipcc is not installed")


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "gemm.s"
    flags = [f for f in B.HIP_FLAGS if f != "-fPIC"]
    cmd = [B.hipcc(), *flags, *B.FILE_FLAGS.get("gemm.hip", []), "--cuda-device-only", "-S",
           "-o", str(out), str(B.CSRC / "gemm.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def _kernels(asm):
    """name -> body (from the symbol's label to its s_endpgm)."""
    out = {}
    for m in re.finditer(r"^(_Z16gemm_wide_kernel\w+):", asm, re.M):
        end = asm.index("s_endpgm", m.end())
        out[m.group(1)] = asm[m.end():end]
    return out


def test_wide_gemm_ring_registers_are_stable(gemm_asm):
    kernels = _kernels(gemm_asm)
    assert kernels, "no gemm_wide_kernel instantiation found"
    for name, body in kernels.items():
        nwv = int(re.search(r"ELi(\d+)E", name).group(1))
        rpt = 512 // (64 * nwv)  # packed words per thread per step (64-row tiles)
        dests = re.findall(r"global_load_(dword|ubyte) (v\d+),", body)
        per_slot = 2 * rpt
        ring = [d for _, d in dests[rpt:]]  # after the row-scale loads
        n_pro = 4 * per_slot
        assert len(ring) >= n_pro + 4 * per_slot + 3 * per_slot, (name, len(ring))
        prologue = ring[:n_pro]
        loop = ring[n_pro:2 * n_pro]
        tail = ring[2 * n_pro:2 * n_pro + 3 * per_slot]
        assert loop == prologue, (name, prologue, loop)
        assert tail == prologue[:3 * per_slot], (name, prologue, tail)
        # every slot's registers are distinct
        assert len(set(prologue)) == len(prologue), (name, prologue)
