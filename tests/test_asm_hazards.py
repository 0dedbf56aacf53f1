"""Generated-code check: no MFMA reads a VGPR that inline asm wrote fewer
than two wait states before, and no inline asm overwrites a VGPR fewer than
seven wait states after an MFMA read it as its accumulator input.

The compiler's hazard recognizer does not count an inline asm statement as
a VALU write, so it keeps no wait states between such a write and an MFMA
that reads the register (gfx950 needs two after a VALU write).  The f16
hi/lo split's v_fma_mixlo/mixhi (common.h) is inline asm and feeds MFMA
operands directly in the attention and fused feed-forward kernels; its asm
blocks end with s_nop 1.  This test compiles every kernel source to gfx950
assembly and scans every MFMA's source registers against the inline asm
writes just before it, so a schedule or helper change cannot bring the
hazard back unnoticed.  (An 8-wave attention variant read stale P
operands this way: its GPU parity test failed until the s_nop was added.)
The other direction: a 16x16 MFMA reads its accumulator input late, so a
VALU write to that register needs seven wait states after the MFMA; the
register allocator hands such a register to the split's first output right
away, so the split's block also starts with an s_nop."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tenzor_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))  # every kernel source
NEED = 2  # wait states between a VALU write and an MFMA read of the register
NEED_WAR = 7  # wait states between a 16x16 MFMA's accumulator read and a VALU write of it


def vgprs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def scan(asm_text, need=NEED):
    """[(line, message)] for each MFMA source register written by inline asm
    fewer than `need` wait states earlier (straight-line look-back)."""
    found, hist, in_asm, func = [], [], False, ""
    for ln, raw in enumerate(asm_text.splitlines(), 1):
        s = raw.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if re.match(r"^_Z\S+:$", s):
            func, hist = s[:-1], []
            continue
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        op = s.split()[0]
        args = [a.strip() for a in s[len(op):].split(",")]
        if op.startswith("v_mfma"):
            srcs = set()
            for a in args[1:4]:
                srcs |= vgprs(a.split()[0]) if a else set()
            waited = 0
            for w, written, asm_write, l2 in reversed(hist):
                if waited >= need:
                    break
                if asm_write and written & srcs:
                    found.append((ln, f"{func}: MFMA reads v{sorted(written & srcs)} written by inline asm at "
                                      f"line {l2}, {waited} wait states before"))
                waited += w
        m = re.match(r"s_nop\s+(\d+)", s)
        w = int(m.group(1)) + 1 if m else 1
        written = vgprs(args[0].split()[0]) if args and args[0] and op.startswith("v_") else set()
        hist.append((w, written, in_asm, ln))
        hist = hist[-16:]
    return found


def scan_war(asm_text, need=NEED_WAR):
    """[(line, message)] for each inline asm VGPR write fewer than `need` wait
    states after an MFMA that read the register as its accumulator input."""
    found, hist, in_asm, func = [], [], False, ""
    for ln, raw in enumerate(asm_text.splitlines(), 1):
        s = raw.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if re.match(r"^_Z\S+:$", s):
            func, hist = s[:-1], []
            continue
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        op = s.split()[0]
        args = [a.strip() for a in s[len(op):].split(",")]
        if in_asm and op.startswith("v_") and args and args[0]:
            written = vgprs(args[0].split()[0])
            waited = 0
            for w, srcc, l2 in reversed(hist):
                if waited >= need:
                    break
                if srcc & written:
                    found.append((ln, f"{func}: inline asm writes v{sorted(srcc & written)} {waited} wait states "
                                      f"after the MFMA at line {l2} read it as its accumulator input"))
                waited += w
        m = re.match(r"s_nop\s+(\d+)", s)
        w = int(m.group(1)) + 1 if m else 1
        srcc = vgprs(args[3].split()[0]) if op.startswith("v_mfma") and len(args) > 3 else set()
        hist.append((w, srcc, ln))
        hist = hist[-32:]
    return found


def test_scanner_flags_a_close_read():
    text = "\n".join([
        "_Zk:",
        ";;#ASMSTART",
        "v_fma_mixhi_f16 v7, -v1, v2, v3 op_sel:[1,0,0] op_sel_hi:[1,0,0]",
        ";;#ASMEND",
        "ds_read_b128 v[10:13], v20",
        "v_mfma_f32_16x16x32_f16 v[0:3], v[10:13], v[4:7], v[0:3]",
    ])
    assert len(scan(text)) == 1
    assert scan(text.replace("ds_read_b128", "s_nop 0\n\tds_read_b128")) == []
    # a compiler-emitted VALU write is the compiler's own business
    assert scan(text.replace(";;#ASMSTART", "").replace(";;#ASMEND", "")) == []
    war = "\n".join([
        "_Zk:",
        "v_mfma_f32_16x16x32_f16 v[0:3], v[4:7], v[8:11], v[12:15]",
        "s_nop 5",
        ";;#ASMSTART",
        "v_fma_mixlo_f16 v12, -v1, v2, v3 op_sel_hi:[1,0,0]",
        ";;#ASMEND",
    ])
    assert len(scan_war(war)) == 1
    assert scan_war(war.replace("s_nop 5", "s_nop 6")) == []


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", SOURCES)
def test_no_mfma_reads_fresh_inline_asm_writes(src, tmp_path):
    from tenzor_amd import build  # the library's own compile flags

    out = tmp_path / (src + ".s")
    cmd = [HIPCC, "-x", "hip", *build.HIPFLAGS, *build.EXTRA_FLAGS.get(src, []), "--cuda-device-only", "-S", "-o",
           str(out), os.path.join(CSRC, src)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    text = out.read_text()
    found = scan(text) + scan_war(text)
    assert not found, "\n".join(msg for _, msg in found[:10])
