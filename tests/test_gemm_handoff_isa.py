"""The GEMM core's x-tile hand-off in compiled code (CPU; needs hipcc).

In `k_gemm` (onecompression_amd/csrc/gemm_core.h), each wave loads part of the next x tile with
LDS-DMA buffer loads. A bare `s_barrier` then hands the tile to every wave. The vmcnt wait before
that barrier must cover the wave's DMA loads. It counts only the vector-memory loads issued after
them, so a load the compiler deletes or moves breaks the count.

The bodies after the loop once relied on prefetch loads the compiler deleted as dead. Up to NW x
loads then stayed in flight across the barrier, which read stale x depending on timing. This test
compiles representative instances to gfx950 assembly. After every run of LDS-DMA loads, the
smallest vmcnt wait before the next s_barrier must be at most the number of vector-memory loads
issued after the run.
"""

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "onecompression_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")

# (BITS, CS, BF16, MT, GROUPED): 2-bit down at 256-row tiles, 4-bit grouped (MoE prefill) at
# 64-row tiles, 8-bit bf16, and the sign GEMM (BITS = 1)
INSTANCES = [(2, 4, "false", 4, "false"), (4, 4, "false", 1, "true"), (8, 1, "true", 2, "false"),
             (1, 4, "false", 4, "false")]


def _asm(tmp_path):
    src = tmp_path / "handoff.hip"
    lines = ['#include "gemm_core.h"']
    for b, cs, bf, mt, gr in INSTANCES:
        lines.append(f"template __global__ void oc_gemm::k_gemm<{b}, {cs}, {bf}, {mt}, {gr}, false>"
                     "(const oc_gemm::GemmArgs);")
    src.write_text("\n".join(lines) + "\n")
    out = tmp_path / "handoff.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S", str(src),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _open_handoffs(asm):
    """(kernel, barriers checked, barriers whose waits leave DMA loads in flight)."""
    found = []
    for m in re.finditer(r"^(_Z\S*k_gemm\S*):", asm, re.M):
        end = asm.index(".Lfunc_end", m.end())
        checked = bad = 0
        state, after, waits = False, 0, []
        for line in asm[m.end():end].split("\n"):
            x = line.strip()
            if not x or x.startswith((".", ";")):
                continue
            op = x.split()[0]
            if op.startswith("buffer_load") and " lds" in x:
                state, after, waits = True, 0, []
                continue
            if not state:
                continue
            if op.startswith(("global_load", "buffer_load")):
                after += 1
            elif op == "s_waitcnt" and "vmcnt" in x:
                waits.append(int(re.search(r"vmcnt\((\d+)\)", x).group(1)))
            elif op == "s_barrier":
                checked += 1
                if not waits or min(waits) > after:
                    bad += 1
                state = False
        found.append((m.group(1), checked, bad))
    return found


def test_every_x_tile_handoff_is_covered(tmp_path):
    found = _open_handoffs(_asm(tmp_path))
    assert len(found) == len(INSTANCES), [f[0] for f in found]
    for name, checked, bad in found:
        assert checked >= 3, (name, checked)  # the loop's three bodies at least
        assert bad == 0, f"{name}: {bad} of {checked} hand-off barriers leave x loads in flight"


def test_checker_flags_an_uncovered_handoff():
    """The checker itself: a barrier after DMA loads with a wait that leaves them in flight."""
    asm = "\n".join([
        "_ZN7oc_gemm6k_gemmIxEEvv:",
        "  buffer_load_dword v1, s[0:3], 0 offen lds",
        "  buffer_load_dword v1, s[0:3], 0 offen lds",
        "  global_load_dwordx2 v[2:3], v[4:5], off",
        "  s_waitcnt vmcnt(6)",
        "  s_barrier",
        "  buffer_load_dword v1, s[0:3], 0 offen lds",
        "  global_load_dwordx2 v[2:3], v[4:5], off",
        "  s_waitcnt vmcnt(1)",
        "  s_barrier",
        ".Lfunc_end0:",
    ])
    assert _open_handoffs(asm) == [("_ZN7oc_gemm6k_gemmIxEEvv", 2, 1)]
