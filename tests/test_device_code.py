"""Wait states around the kernels' inline assembly, checked in the compiler's gfx950 output.

The compiler inserts the wait states the hardware needs between its own instructions, but it
cannot see inside an inline-assembly statement. Two rules matter for the statements these
kernels use (the compiler applies the same numbers to its own code):
  - a VGPR written inside inline assembly must not be read by a matrix-core instruction fewer
    than 2 wait states later (the compiler pads its own VALU -> MFMA operand writes with s_nop 1);
  - a vector-memory instruction inside inline assembly (the LDS DMA global_load_lds_dwordx4)
    must not read an SGPR that a VALU instruction wrote fewer than 5 wait states earlier, nor M0
    fewer than 1 wait state after an SALU write to it.
The sources are compiled to device assembly (hipcc -S) with the library's flags; CPU only.

One more rule comes from the compiler itself: v_dot2c_f32_bf16 must take its constant bf16 pairs
from registers. As an inline constant the compiler encodes the pair (-1, 0) as -1.0, which the
instruction reads as the 32-bit pattern 0xbf800000, i.e. the pair (0, -1).
"""

import os
import re
import shutil
import subprocess

import pytest

from llmario_amd import build as B

DEVICE_SOURCES = ["prefill.hip", "decode.hip", "kv_kernels.hip"]


_ASM = {}   # source -> assembly lines (each source compiled once per session)


def _asm(src, tmp_path):
    if src in _ASM:
        return _ASM[src]
    out = tmp_path / (src + ".s")
    cmd = [B.HIPCC, *B.FLAGS, *B.EXTRA.get(src, []), "-x", "hip", "--cuda-device-only", "-S",
           os.path.join(B.CSRC, src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    _ASM[src] = out.read_text().splitlines()
    return _ASM[src]


def _vregs(op):
    m = re.match(r"-?v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"-?v(\d+)$", op)
    return {int(m.group(1))} if m else set()


def _sregs(op):
    if op in ("m0", "vcc", "vcc_lo", "vcc_hi", "exec"):
        return {op}
    m = re.match(r"s\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", op)
    return {int(m.group(1))} if m else set()


def _instructions(lines):
    """(function, inside inline asm, opcode, operands) per instruction, in order."""
    fn, in_asm = "", False
    for line in lines:
        t = line.strip()
        if re.match(r"^_Z\S+:", line):
            fn = line.split(":")[0]
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not t or t.startswith((".", ";")) or t.endswith(":"):
            continue
        op, _, rest = t.partition(" ")
        ops = [o.strip() for o in rest.split(";")[0].split(",")] if rest else []
        yield fn, in_asm, op, ops


def _wait_states(op, ops):
    return int(ops[0]) + 1 if op == "s_nop" and ops else 1


def _scan(lines):
    problems = []
    vgpr_w = []   # (regs, wait states since, function): VGPRs written inside inline asm
    sgpr_w = []   # (regs, wait states since): SGPRs written by VALU instructions
    m0_w = []     # wait states since an SALU write to M0
    fn_prev = None
    for fn, in_asm, op, ops in _instructions(lines):
        if fn != fn_prev:
            vgpr_w, sgpr_w, m0_w, fn_prev = [], [], [], fn
        if "mfma" in op and len(ops) >= 3:
            srcs = set().union(*(_vregs(o) for o in ops[1:]))
            for regs, w in vgpr_w:
                if regs & srcs and w < 2:
                    problems.append(f"{fn}: inline-asm VGPR write read by {op} after {w} wait states")
        if in_asm and (op.startswith(("global_", "buffer_", "flat_", "scratch_"))):
            srcs = set().union(*(_sregs(o) for o in ops[1:])) if len(ops) > 1 else set()
            for regs, w in sgpr_w:
                if regs & srcs and w < 5:
                    problems.append(f"{fn}: {op} reads an SGPR a VALU instruction wrote {w} wait states before")
            if "lds" in op:
                for w in m0_w:
                    if w < 1:
                        problems.append(f"{fn}: {op} reads M0 {w} wait states after an SALU write")
        ws = _wait_states(op, ops)
        vgpr_w = [(r, w + ws) for r, w in vgpr_w if w + ws < 8]
        sgpr_w = [(r, w + ws) for r, w in sgpr_w if w + ws < 8]
        m0_w = [w + ws for w in m0_w if w + ws < 8]
        if in_asm and op.startswith("v_") and ops:
            vgpr_w.append((_vregs(ops[0]), 0))
        if op.startswith("v_") and ops and _sregs(ops[0]):
            sgpr_w.append((_sregs(ops[0]), 0))
        if op.startswith("s_") and ops and ops[0] == "m0":
            m0_w.append(0)
    return problems


@pytest.mark.skipif(not os.path.exists(B.HIPCC) and shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("src", DEVICE_SOURCES)
def test_inline_asm_wait_states(src, tmp_path):
    problems = _scan(_asm(src, tmp_path))
    assert not problems, "\n".join(problems[:20])


@pytest.mark.skipif(not os.path.exists(B.HIPCC) and shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("src", DEVICE_SOURCES)
def test_bf16_dot2_sources_are_registers(src, tmp_path):
    bad = []
    for fn, _, op, ops in _instructions(_asm(src, tmp_path)):
        if op.startswith("v_dot2") and "bf16" in op and any(not _vregs(o) for o in ops[1:]):
            bad.append(f"{fn}: {op} {', '.join(ops)}")
    assert not bad, "\n".join(bad[:10])


def test_dot2_check_flags_a_constant_pair():
    lines = ["_Zk:", "\tv_dot2c_f32_bf16_e32 v0, -1.0, v2", "\tv_dot2c_f32_bf16_e32 v1, v7, v5"]
    flagged = [op for _, _, op, ops in _instructions(lines) if op.startswith("v_dot2") and any(not _vregs(o) for o in ops[1:])]
    assert flagged == ["v_dot2c_f32_bf16_e32"]


def test_scanner_flags_a_short_wait():
    """The scanner itself: a DMA right after a v_readfirstlane of its base, an MFMA right after an
    asm write of its operand, and the padded forms that pass."""
    bad = """_Zk:
\tv_readfirstlane_b32 s8, v4
\t;;#ASMSTART
\ts_mov_b32 m0, s3
\tglobal_load_lds_dwordx4 v9, s[8:9]
\t;;#ASMEND
\t;;#ASMSTART
\tv_fma_mixlo_f16 v10, v1, v2, 0
\t;;#ASMEND
\tv_mfma_f32_16x16x16_f16 v[20:23], v[10:11], v[12:13], v[20:23]
""".splitlines()
    found = _scan(bad)
    assert any("SGPR" in p for p in found) and any("M0" in p for p in found) and any("mfma" in p for p in found)
    good = """_Zk:
\tv_readfirstlane_b32 s8, v4
\t;;#ASMSTART
\ts_nop 4
\ts_mov_b32 m0, s3
\ts_nop 0
\tglobal_load_lds_dwordx4 v9, s[8:9]
\t;;#ASMEND
\t;;#ASMSTART
\tv_fma_mixlo_f16 v10, v1, v2, 0
\t;;#ASMEND
\ts_nop 1
\tv_mfma_f32_16x16x16_f16 v[20:23], v[10:11], v[12:13], v[20:23]
""".splitlines()
    assert _scan(good) == []
