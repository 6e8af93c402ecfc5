"""Static check of the inline-asm LDS / global loads in the HIP sources.

Some fragment and input loads are inline asm, invisible to the compiler's
wait-count pass; the code waits for them with an asm `s_waitcnt` whose
operands are tied to the loaded registers. That is only correct if the
compiled code never reads, writes or copies such a register between the load
and the next asm wait. This test compiles the sources to gfx950 assembly
(hipcc, device only) and scans every kernel for such an access. CPU only;
skipped where hipcc is absent.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "torchplusplus_amd", "csrc")
SOURCES = ["attention.hip", "gemv.hip"]

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out |= {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
        else:
            out.add(f"{m.group(4)}{m.group(5)}")
    return out


def scan(asm_text):
    """(number of asm loads, list of offending lines). A register loaded by an
    asm ds_read / global_load is pending until the next asm s_waitcnt; any
    compiler-generated instruction naming it meanwhile is an offence."""
    pending, in_asm, loads, bad, func = set(), False, 0, [], ""
    for line in asm_text.split("\n"):
        t = line.strip()
        if re.match(r"^_Z\w+:", t):
            func, pending = t, set()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not t or t.startswith(";") or t.startswith(".") or t.endswith(":"):
            continue
        ins = t.split()[0]
        if in_asm:
            if ins.startswith("s_waitcnt"):
                pending = set()
            elif ins.startswith("ds_read") or ins.startswith("global_load"):
                pending |= _regs(t.split(None, 1)[1].split(",")[0])
                loads += 1
            continue
        if ins == "s_endpgm":
            pending = set()
            continue
        if pending and " " in t and _regs(t.split(None, 1)[1]) & pending:
            bad.append(f"{func[:60]}: {t}")
    return loads, bad


def test_scan_flags_an_early_use():
    """The scanner itself: a use between the asm load and its wait is caught,
    a use after the wait is not."""
    early = ";;#ASMSTART\n\tds_read_b128 v[4:7], v1\n;;#ASMEND\n\tv_mov_b32 v9, v5\n"
    late = early.replace("\tv_mov_b32 v9, v5\n", ";;#ASMSTART\n\ts_waitcnt lgkmcnt(0)\n;;#ASMEND\n\tv_mov_b32 v9, v5\n")
    assert scan(early)[1] and not scan(late)[1]


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not installed")
def test_no_access_to_asm_loaded_registers_before_their_wait():
    flags = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
             "--cuda-device-only", "-S"]
    with tempfile.TemporaryDirectory() as tmp:
        procs = []
        for src in SOURCES:
            out = os.path.join(tmp, src + ".s")
            procs.append((src, out, subprocess.Popen(["hipcc", *flags, os.path.join(CSRC, src), "-o", out],
                                                     stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)))
        for src, out, p in procs:
            _, err = p.communicate(timeout=600)
            assert p.returncode == 0, f"{src}: {err.decode()[-2000:]}"
            loads, bad = scan(open(out).read())
            assert loads > 0, f"{src}: no inline-asm loads found"
            assert not bad, f"{src}: registers touched before their wait:\n" + "\n".join(bad[:10])
