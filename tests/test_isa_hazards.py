"""CPU test over the gfx950 machine code of every kernel source: no vector-memory instruction reads an SGPR that a
VALU instruction wrote fewer than 5 wait states before it.

GFX9-family hardware (gfx950 included) needs 5 wait states between a VALU write of an SGPR (v_readfirstlane,
v_readlane, a v_cmp into an SGPR pair) and a vector-memory instruction that reads that SGPR (a buffer descriptor, a
scalar offset or base).  The compiler inserts them for the instructions it generates, but not for inline assembly:
the direct-to-LDS copies are inline assembly whose descriptor words come from v_readfirstlane, and with fewer wait
states such a copy may use stale descriptor words (a wrong base or range, i.e. an access outside its buffer).

The test compiles each source to assembly with the library's own flags (hipcc --cuda-device-only -S; no GPU needed)
and walks back from every vector-memory instruction with SGPR operands, counting wait states (one per instruction,
N + 1 for s_nop N), until 5 are reached or a VALU write of one of its SGPRs is found.
"""
from __future__ import annotations

import importlib.util
import os
import re
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen3.8-flash-next-24gb-sglang_amd")

_VMEM = ("buffer_", "global_", "flat_", "scratch_")
_WAIT_STATES = 5


def _build_module():
    spec = importlib.util.spec_from_file_location("_kvt_build_isa", os.path.join(PKG, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _sgprs(text: str) -> set:
    regs = set()
    for m in re.finditer(r"\bs\[(\d+):(\d+)\]", text):
        regs |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"(?<![\w\[])s(\d+)\b", text):
        regs.add(int(m.group(1)))
    return regs


def _valu_sgpr_dest(line: str) -> set:
    m = re.match(r"(v_\w+)\s+(s\[(\d+):(\d+)\]|s(\d+))\b", line)
    if m is None:
        return set()
    if m.group(3) is not None:
        return set(range(int(m.group(3)), int(m.group(4)) + 1))
    return {int(m.group(5))}


def hazards(asm_lines) -> tuple:
    """(vector-memory instructions with SGPR operands, list of (VALU write, memory instruction, wait states))."""
    lines = []
    for raw in asm_lines:
        text = raw.split(";")[0].strip()
        if text and not text.startswith(".") and not text.endswith(":"):
            lines.append(text)
    checked, found = 0, []
    for i, line in enumerate(lines):
        if not line.startswith(_VMEM):
            continue
        operands = line.split(None, 1)[1] if " " in line else ""
        regs = _sgprs(operands)
        if not regs:
            continue
        checked += 1
        ws, k = 0, i - 1
        while k >= 0 and ws < _WAIT_STATES:
            prev = lines[k]
            if _valu_sgpr_dest(prev) & regs:
                found.append((prev, line, ws))
                break
            nop = re.match(r"s_nop\s+(\d+)", prev)
            ws += int(nop.group(1)) + 1 if nop else 1
            k -= 1
    return checked, found


def test_scanner_flags_a_short_distance():
    """The walk-back finds a VALU SGPR write 2 wait states before a buffer load that reads it, and accepts one
    that s_nop 4 separates from the load."""
    bad = ["v_readfirstlane_b32 s22, v11", "s_mov_b32 m0, s8", "s_nop 0",
           "buffer_load_dwordx4 v15, s[20:23], 0 offen nt lds"]
    good = ["v_readfirstlane_b32 s22, v11", "s_mov_b32 m0, s8", "s_nop 4",
            "buffer_load_dwordx4 v15, s[20:23], 0 offen nt lds"]
    other = ["v_readfirstlane_b32 s40, v11", "buffer_load_dwordx4 v15, s[20:23], 0 offen nt lds"]
    assert len(hazards(bad)[1]) == 1
    assert hazards(good)[1] == []
    assert hazards(other)[1] == []


def test_no_valu_sgpr_to_vmem_hazard_in_any_kernel():
    b = _build_module()
    if not os.path.exists(b.HIPCC):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as tmp:
        def asm(src):
            out = os.path.join(tmp, os.path.basename(src) + ".s")
            cmd = [b.HIPCC, *b.CFLAGS, *b.EXTRA_CFLAGS.get(os.path.basename(src), []), "--cuda-device-only", "-S",
                   src, "-o", out]
            res = subprocess.run(cmd, capture_output=True, text=True)
            assert res.returncode == 0, res.stderr[-2000:]
            with open(out) as f:
                return os.path.basename(src), f.readlines()

        with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
            results = list(ex.map(asm, b.sources()))
    total = 0
    for name, lines in results:
        checked, found = hazards(lines)
        total += checked
        assert not found, f"{name}: VALU SGPR write within {_WAIT_STATES} wait states of a memory read: {found[:3]}"
    assert total > 0
