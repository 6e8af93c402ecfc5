"""Static check of the inline-asm LDS / global loads in the HIP sources.

Some fragment and input loads are inline asm, invisible to the compiler's
wait-count pass; the code waits for them with an asm `s_waitcnt` whose
operands are tied to the loaded registers. That is only correct if the
compiled code never reads, writes or copies such a register between the load
and the next asm wait, and if a counted wait `s_waitcnt vmcnt(N)` leaves in
flight only instructions issued after the asm loads (loads complete in issue
order: at least N vector-memory instructions must follow the last asm load).
This test compiles the sources to gfx950 assembly (hipcc, device only) and
scans every kernel for both. CPU only; skipped where hipcc is absent.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "torchplusplus_amd", "csrc")
SOURCES = ["attention.hip", "gemv.hip", "ffn.hip"]

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out |= {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
        else:
            out.add(f"{m.group(4)}{m.group(5)}")
    return out


_BRANCH = re.compile(r"^s_(c?branch\w*)\s+(\.LBB\w+)")


def _lines(asm_text):
    """(kind, text) per line: 'func' / 'label' / 'asm' / 'ins', in order."""
    in_asm = False
    for line in asm_text.split("\n"):
        t = line.strip()
        if re.match(r"^_Z\w+:", t):
            yield "func", t
            continue
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if re.match(r"^\.LBB\w+:", t):
            yield "label", t[:-1]
            continue
        if not t or t.startswith(";") or t.startswith(".") or t.endswith(":"):
            continue
        yield ("asm" if in_asm else "ins"), t


def scan(asm_text):
    """(number of asm loads, list of offending lines). A register loaded by an
    asm ds_read / global_load is pending until the next asm s_waitcnt; any
    compiler-generated instruction naming it meanwhile is an offence. The
    pending set follows forward branches: at a label it is the union of the
    fall-through state and that of every branch to it (after an s_branch
    nothing falls through)."""
    pending, loads, bad, func, at_label, live = set(), 0, [], "", {}, True
    for kind, t in _lines(asm_text):
        if kind == "func":
            func, pending, at_label, live = t, set(), {}, True
            continue
        if kind == "label":
            pending = (pending if live else set()) | at_label.pop(t, set())
            live = True
            continue
        ins = t.split()[0]
        if kind == "asm":
            if ins.startswith("s_waitcnt"):
                pending = set()
            elif ins.startswith("ds_read") or ins.startswith("global_load"):
                pending |= _regs(t.split(None, 1)[1].split(",")[0])
                loads += 1
            continue
        if ins == "s_endpgm":
            pending, live = set(), False
            continue
        b = _BRANCH.match(t)
        if b:
            at_label[b.group(2)] = at_label.get(b.group(2), set()) | pending
            if b.group(1) == "branch":
                live = False
            continue
        if pending and " " in t and _regs(t.split(None, 1)[1]) & pending:
            bad.append(f"{func[:60]}: {t}")
    return loads, bad


_VMEM = re.compile(r"^(global_|buffer_|flat_|scratch_)")


def vm_counts(asm_text):
    """(number of counted asm waits checked, list of offences). After an asm
    global_load, an asm `s_waitcnt vmcnt(N)` covers the asm loads only if at
    least N vector-memory instructions (loads, LDS-DMA, stores, atomics)
    were issued after the last of them on every path to the wait (forward
    branches followed as in scan; the fewest over the merging paths)."""
    after, checked, bad, func, at_label, live = None, 0, [], "", {}, True

    def merge(a, b):
        return b if a is None else a if b is None else min(a, b)

    for kind, t in _lines(asm_text):
        if kind == "func":
            func, after, at_label, live = t, None, {}, True
            continue
        if kind == "label":
            after = merge(after if live else None, at_label.pop(t, None))
            live = True
            continue
        ins = t.split()[0]
        if kind == "asm":
            if ins.startswith("global_load"):
                after = 0
            elif ins.startswith("s_waitcnt"):
                m = re.search(r"vmcnt\((\d+)\)", t)
                if m and after is not None:
                    checked += 1
                    if after < int(m.group(1)):
                        bad.append(f"{func[:60]}: {t} with {after} vector-memory instructions after the loads")
                if m:
                    after = None
            continue
        if ins == "s_endpgm":
            after, live = None, False
            continue
        br = _BRANCH.match(t)
        if br:
            at_label[br.group(2)] = merge(at_label.get(br.group(2)), after)
            if br.group(1) == "branch":
                live = False
            continue
        if after is not None and _VMEM.match(ins):
            after += 1
    return checked, bad


def test_vm_count_check_flags_a_short_wait():
    """The count check itself: vmcnt(2) after one later load is too few."""
    body = (";;#ASMSTART\n\tglobal_load_dwordx4 v[4:7], v[0:1], off\n;;#ASMEND\n"
            "\tglobal_load_lds_dwordx4 v[2:3], off\n;;#ASMSTART\n\ts_waitcnt vmcnt({n})\n;;#ASMEND\n")
    assert vm_counts(body.format(n=2))[1] and not vm_counts(body.format(n=1))[1]


def test_scan_flags_an_early_use():
    """The scanner itself: a use between the asm load and its wait is caught,
    a use after the wait is not, a use on a path that branched away before
    the load is not, and a use after a branch merge with a pending path is."""
    early = ";;#ASMSTART\n\tds_read_b128 v[4:7], v1\n;;#ASMEND\n\tv_mov_b32 v9, v5\n"
    late = early.replace("\tv_mov_b32 v9, v5\n", ";;#ASMSTART\n\ts_waitcnt lgkmcnt(0)\n;;#ASMEND\n\tv_mov_b32 v9, v5\n")
    assert scan(early)[1] and not scan(late)[1]
    other_path = ("\ts_cbranch_scc1 .LBB0_2\n;;#ASMSTART\n\tds_read_b128 v[4:7], v1\n;;#ASMEND\n"
                  "\ts_branch .LBB0_3\n.LBB0_2:\n\tv_mov_b32 v5, 0\n.LBB0_3:\n"
                  ";;#ASMSTART\n\ts_waitcnt lgkmcnt(0)\n;;#ASMEND\n")
    assert not scan(other_path)[1]
    merged = other_path.replace(".LBB0_3:\n;;", ".LBB0_3:\n\tv_mov_b32 v9, v6\n;;")
    assert scan(merged)[1]


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
            text = open(out).read()
            loads, bad = scan(text)
            assert loads > 0, f"{src}: no inline-asm loads found"
            assert not bad, f"{src}: registers touched before their wait:\n" + "\n".join(bad[:10])
            checked, short = vm_counts(text)
            if src != "attention.hip":  # its asm loads are LDS reads (lgkmcnt waits)
                assert checked > 0, f"{src}: no counted wait after asm global loads found"
            assert not short, f"{src}: counted waits that could release early:\n" + "\n".join(short[:10])
