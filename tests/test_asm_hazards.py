"""Wait states around hand-written instructions (CPU; needs hipcc).

The compiler inserts the wait states gfx950 needs between instructions it
generates, but it does not look inside inline asm text. The library's asm
(the fp16 widening's SDWA conversions, the LDS DMA with its M0 write) must
therefore carry its own. This test compiles every library source to gfx950
assembly, exactly as the library is built, and checks three rules over every
instruction, the compiler's own and the asm's alike (the compiler's code
meets them by construction, so a hit is hand-written):

- an LDS DMA (``global_load_lds_*``) is at least one wait state after the last
  write of M0, whose LDS address it reads;
- a VALU instruction that reads or writes a VGPR is at least one wait state
  after an SDWA write of part of it (``dst_sel`` WORD / BYTE), including the
  implicit read of a preserving SDWA write;
- an MFMA that reads a VGPR as its A or B operand is at least two wait states
  after a VALU (non-MFMA) write of it.

Wait states count instructions in program order (``s_nop n`` counts n + 1)
within straight-line code; every label starts afresh.
"""
from __future__ import annotations

import concurrent.futures
import re
import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

from cublade_amd import _abi, _loader

_VREG = re.compile(r"v\[(\d+):(\d+)\]$|v(\d+)$")


def _vregs(tok: str) -> set[int]:
    m = _VREG.match(tok.strip().split(" ")[0]) if tok.strip() else None
    if not m:
        return set()
    if m.group(3) is not None:
        return {int(m.group(3))}
    return set(range(int(m.group(1)), int(m.group(2)) + 1))


def scan(asm_text: str) -> list[tuple[str, int, str]]:
    """(function, line, rule) of every instruction that breaks a rule."""
    bad = []
    fn = "?"
    clock = 0
    m0_at = None
    sdwa_at: dict[int, int] = {}
    valu_at: dict[int, int] = {}
    for n, line in enumerate(asm_text.splitlines(), 1):
        s = line.split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        if s.endswith(":"):
            if not s.startswith(".L"):
                fn = s[:-1]
            m0_at, sdwa_at, valu_at = None, {}, {}
            continue
        op, _, rest = s.partition(" ")
        ops = [o.strip() for o in rest.split(",")] if rest else []
        nop = re.match(r"s_nop\s+(\d+)", s)
        clock += int(nop.group(1)) + 1 if nop else 1
        if nop:
            continue
        if op.startswith("global_load_lds") or (op.startswith("buffer_load") and " lds" in s):
            if m0_at is not None and clock - m0_at - 1 < 1:
                bad.append((fn, n, "M0 write -> LDS DMA"))
        if op.startswith("v_"):
            touched = set()
            for o in ops:
                touched |= _vregs(o)
            if any(r in sdwa_at and clock - sdwa_at[r] - 1 < 1 for r in touched):
                bad.append((fn, n, "SDWA sub-dword write -> VALU"))
        if op.startswith("v_mfma"):
            ab = _vregs(ops[1]) | _vregs(ops[2])
            if any(r in valu_at and clock - valu_at[r] - 1 < 2 for r in ab):
                bad.append((fn, n, "VALU write -> MFMA A/B read"))
        if ops and ops[0].split(" ")[0] == "m0":
            m0_at = clock
        if op.startswith("v_") and ops:
            for r in _vregs(ops[0]):
                sdwa_at.pop(r, None)
                valu_at.pop(r, None)
                if not op.startswith(("v_mfma", "v_accvgpr")):
                    valu_at[r] = clock
                if "_sdwa" in op and re.search(r"dst_sel:(WORD|BYTE)", s):
                    sdwa_at[r] = clock
    return bad


def test_scan_flags_each_rule():
    """The scanner itself: one violation of each rule, and the fixed forms."""
    bad = scan("k:\n"
               "s_mov_b32 m0, s4\n"
               "global_load_lds_dwordx4 v1, s[0:1]\n"
               "v_cvt_f16_i16_sdwa v2, sext(v1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n"
               "v_cvt_f16_i16_sdwa v2, sext(v1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n"
               "s_nop 0\n"
               "v_mfma_f32_32x32x16_f16 v[10:25], v[2:5], v[6:9], 0\n")
    assert [r for _, _, r in bad] == ["M0 write -> LDS DMA", "SDWA sub-dword write -> VALU",
                                      "VALU write -> MFMA A/B read"]
    assert scan("k:\n"
                "s_mov_b32 m0, s4\n"
                "s_nop 0\n"
                "global_load_lds_dwordx4 v1, s[0:1]\n"
                "v_cvt_f16_i16_sdwa v2, sext(v1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n"
                "v_cvt_f16_i16_sdwa v3, sext(v1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n"
                "v_cvt_f16_i16_sdwa v2, sext(v1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n"
                "v_cvt_f16_i16_sdwa v3, sext(v1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3\n"
                "s_nop 1\n"
                "v_mfma_f32_32x32x16_f16 v[10:25], v[2:5], v[6:9], 0\n") == []


def _device_asm(src: Path, out: Path) -> str:
    flags = [f for f in _loader.BASE_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [_loader.hipcc(), f"--offload-arch={_loader.DEFAULT_ARCH}", *flags,
           f"-I{_loader.INCLUDE}", f"-I{_loader.CSRC}", "-S", "--cuda-device-only",
           str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_library_asm_wait_states():
    sources = [Path(s) for s in _abi.SOURCES if str(s).endswith(".hip")]
    assert sources
    with tempfile.TemporaryDirectory() as td, \
            concurrent.futures.ThreadPoolExecutor(max_workers=4) as pool:
        texts = pool.map(lambda s: (s.name, _device_asm(s, Path(td) / (s.stem + ".s"))), sources)
        problems = []
        n_asm = 0
        for name, text in texts:
            n_asm += text.count(";;#ASMSTART")
            problems += [(name, *b) for b in scan(text)]
    assert n_asm > 0, "no inline asm found: the scan would check nothing hand-written"
    assert not problems, f"{len(problems)} wait-state violations, first: {problems[:5]}"
