"""DPP read-after-VALU-write hazards in the compiled backward kernels.

A DPP instruction that reads a VGPR needs two wait states after a VALU
instruction that wrote it; the compiler inserts them for the DPP it emits
itself, but not for DPP written as inline assembly, whose contents it does not
see.  The backward's inline DPP instructions are `bc_fmac` (ss_common.cuh),
whose source is a block register read from LDS and so carries no wait states
of its own, and the masked reduce-scatter folds (scan_bwd.hip), which do.
This test compiles scan_bwd.hip for gfx950 with the library's flags and checks
every DPP instruction of the assembly: no VALU write of its DPP source in the
two wait states before it, and no label in that window (its predecessors are
not visible, so that counts as a failure too).  CPU only: it needs hipcc, not
a GPU.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from ssm_mamba_amd import _build as B


def _vregs(op):
    op = op.strip().rstrip(",")
    m = re.match(r"v\[(\d+):(\d+)\]$", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op)
    return {int(m.group(1))} if m else set()


def dpp_hazards(asm):
    """(DPP instructions checked, list of hazards) over assembly text."""
    lines = asm.splitlines()
    hazards, checked = [], 0
    for i, ln in enumerate(lines):
        s = ln.split(";")[0].strip()
        if not re.match(r"v_\w+_dpp\s", s):
            continue
        ops = s.split(None, 1)[1].split(",")
        src = _vregs(ops[1])  # the DPP operand is the first source
        checked += 1
        waits, j = 0, i - 1
        while waits < 2 and j >= 0:
            p = lines[j].split(";")[0].strip()
            j -= 1
            if not p or (p.startswith(".") and not re.match(r"\.L\w+:", p)):
                continue
            if p.endswith(":"):
                hazards.append((i + 1, s, "label " + p))
                break
            m = re.match(r"s_nop\s+(\d+)", p)
            if m:
                waits += int(m.group(1)) + 1
                continue
            waits += 1
            if p.startswith("v_"):
                name, rest = (p.split(None, 1) + [""])[:2]
                pops = rest.split(",")
                written = _vregs(pops[0]) if pops else set()
                if "permlane" in name and len(pops) > 1:
                    written |= _vregs(pops[1])  # the swaps write both operands
                if written & src:
                    hazards.append((i + 1, s, p))
                    break
    return checked, hazards


def test_checker_finds_a_planted_hazard():
    ok = "v_mul_f32_e32 v3, v4, v5\ns_nop 1\nv_add_f32_dpp v1, v3, v3 row_ror:8 row_mask:0xf\n"
    bad = "v_mul_f32_e32 v3, v4, v5\nv_add_f32_dpp v1, v3, v3 row_ror:8 row_mask:0xf\n"
    far = "v_mul_f32_e32 v3, v4, v5\nv_mov_b32 v7, v8\nv_mov_b32 v9, v8\nv_add_f32_dpp v1, v3, v3 quad_perm:[1,0,3,2]\n"
    label = ".LBB0_1:\nv_fmac_f32_dpp v1, v3, v2 row_newbcast:3 row_mask:0xf\n"
    swap = "v_permlane16_swap_b32_e32 v6, v3\nv_add_f32_dpp v1, v3, v3 row_ror:8\n"
    assert dpp_hazards(ok) == (1, [])
    assert len(dpp_hazards(bad)[1]) == 1
    assert dpp_hazards(far) == (1, [])
    assert len(dpp_hazards(label)[1]) == 1
    assert len(dpp_hazards(swap)[1]) == 1


@pytest.mark.timeout(600)
def test_backward_kernels_have_no_dpp_hazard():
    if not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "scan_bwd.s")
        cmd = [B.hipcc(), *B.COMMON_FLAGS, *B.DEVICE_FLAGS, "--cuda-device-only", "-S",
               os.path.join(B.CSRC, "scan_bwd.hip"), "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-3000:]
        with open(out) as f:
            checked, hazards = dpp_hazards(f.read())
    assert checked > 1000, checked
    assert not hazards, hazards[:5]
