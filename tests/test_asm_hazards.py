"""Wait states before the direct-to-LDS loads (CPU only: compiles, runs nothing).

The GEMM and attention kernels stage operands with buffer_load_dwordx4 ...
lds issued from inline assembly (lz_dma16 in csrc/lz_common.h); the load
reads its buffer descriptor and scalar offset from SGPRs.  On CDNA, a VALU
instruction that writes an SGPR (v_readfirstlane_b32, v_readlane_b32, a
VOP3 compare into an SGPR pair) must be followed by 5 wait states before a
VMEM instruction reads that SGPR, and the compiler does not pad for
instructions inside inline assembly.  Without them the load can use the
SGPR's previous value, i.e. a stale or garbage address.  This test compiles
every source that issues such loads to gfx950 assembly with the library's
own flags and checks each load against the instructions before it.
"""
from __future__ import annotations

import concurrent.futures as cf
import re
import subprocess
import sys
import tempfile
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "cs244c-llama-zero_amd" / "csrc"
sys.path.insert(0, str(CSRC))
import build as B  # noqa: E402  (csrc/build.py: the library's compiler flags)

SOURCES = ["gemm.hip", "attn.hip"]  # the sources that call lz_dma16
WAIT_STATES = 5


def _sgprs(tok: str) -> set:
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _instructions(asm: str):
    """(function, instruction text or None at a function's start) in order."""
    fn = None
    for line in asm.splitlines():
        t = line.split(";")[0].strip()
        if re.match(r"^_Z\S+:$", t):
            fn = t[:-1]
            yield fn, None
            continue
        if not t or t.startswith(".") or t.endswith(":"):
            continue
        yield fn, t


def hazards(asm: str):
    """Loads `buffer_load* ... lds` whose descriptor or scalar offset was
    written by a VALU instruction fewer than WAIT_STATES wait states before
    (each instruction counts one, s_nop N counts N + 1; walks back through
    straight-line code, so a loop's back edge is not followed).  Returns
    (number of loads, list of (function, writer, load))."""
    insts = list(_instructions(asm))
    found, loads = [], 0
    for i, (fn, t) in enumerate(insts):
        if t is None or not (t.startswith("buffer_load") and t.endswith(" lds")):
            continue
        loads += 1
        operands = [o.strip() for o in t.split(None, 1)[1].split(",")]
        reads = set()
        for o in operands[1:3]:  # the descriptor and the scalar offset
            reads |= _sgprs(o)
        ws, j = 0, i - 1
        while j >= 0 and ws < WAIT_STATES and insts[j][1] is not None:
            u = insts[j][1]
            if u.startswith("v_") and " " in u:
                dst = u.split(None, 1)[1].split(",")[0].strip()
                if _sgprs(dst) & reads:
                    found.append((fn, u, t))
                    break
            m = re.match(r"s_nop\s+(\d+)", u)
            ws += int(m.group(1)) + 1 if m else 1
            j -= 1
    return loads, found


def test_the_scan_flags_a_readfirstlane_right_before_a_load():
    asm = "\n".join([
        "_Zkernel:",
        "v_readfirstlane_b32 s1, v229",
        "v_readfirstlane_b32 s0, v228",
        "s_mov_b32 m0, s23",
        "s_nop 0",
        "buffer_load_dwordx4 v235, s[0:3], s20 offen lds",
        "v_readfirstlane_b32 s4, v1",
        "s_nop 4",
        "buffer_load_dwordx4 v236, s[4:7], s20 offen lds",
    ])
    loads, found = hazards(asm)
    assert loads == 2 and len(found) == 1 and found[0][1].startswith("v_readfirstlane_b32 s0")


def _device_asm(hipcc: str, src: Path, out: Path) -> tuple[str, int, str]:
    cmd = [hipcc, "--offload-arch=gfx950", *B.COMMON_FLAGS, *B.EXTRA_FLAGS.get(src.name, []), "--cuda-device-only",
           "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    return src.name, proc.returncode, proc.stderr[-2000:]


def test_direct_to_lds_loads_have_their_wait_states():
    try:
        hipcc = B.find_hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as td:
        outs = {s: Path(td) / (Path(s).stem + ".s") for s in SOURCES}
        with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
            results = list(pool.map(lambda s: _device_asm(hipcc, CSRC / s, outs[s]), SOURCES))
        for name, rc, err in results:
            assert rc == 0, f"{name}: {err}"
        total = 0
        for s in SOURCES:
            loads, found = hazards(outs[s].read_text())
            assert not found, f"{s}: {found[:3]}"
            total += loads
    assert total > 0  # the scan saw the loads it is meant to check
