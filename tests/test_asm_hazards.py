"""Wait states after the inline-asm MFMAs of the gfx950 kernels (CPU: compiles to assembly).

Accumulators that only MFMAs touch (dQ, dK, dV, O) are accumulated in place through inline asm
(`mfma_acc` in csrc/common.h, the accumulator tied to the output), which the compiler's hazard
recognizer cannot see into.  The ISA requires an MFMA's passes plus a few wait states before
another unit reads (or overwrites) its destination registers; the kernels meet that with
`mfma_drain` (20 wait states) before their own reads.  If register allocation ever copies or
reads such an accumulator with a compiler-emitted instruction sooner, that instruction sees a
stale value and the result is wrong only now and then, under load.  This test compiles the
library to gfx950 assembly with the build flags and checks that every compiler-emitted
instruction touching the destination of an inline-asm MFMA comes at least 20 wait states after
it (`s_nop N` counts N + 1, any other instruction 1), scanning each kernel in fall-through
order.  In the other direction, an inline-asm MFMA must not read an A or B operand that a
compiler-emitted VALU instruction wrote fewer than 2 wait states before (the schedules that drop
`mfma_acc`'s leading `s_nop 1` rely on this).  M0 is a register the compiler reserves: an inline
asm block that writes M0 must save it first and put the saved value back as its last M0 write (the
LDS-DMA copy takes M0 as an input operand and writes none).  A VMEM instruction that reads an SGPR
needs 5 wait states after a VALU instruction wrote it (the copy's buffer descriptor comes from
v_readfirstlane): every inline-asm LDS-DMA copy is checked for that, walking back from the copy
over every path into it.  Each scan is checked on a planted case."""
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NEED = 20


def _regs(tok):
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def early_touches(asm_text):
    """(kernel, line, wait states, instruction) for compiler-emitted instructions that touch an
    inline-asm MFMA's destination registers fewer than NEED wait states after it."""
    found = []
    kern, inasm, pending = None, False, []  # pending: [dest regs, wait states since]
    for i, line in enumerate(asm_text.split("\n")):
        t = line.strip()
        m = re.match(r"^(_Z\w+):", t)
        if m:
            kern, pending = m.group(1), []
            continue
        if t.startswith(";;#ASMSTART"):
            inasm = True
            continue
        if t.startswith(";;#ASMEND"):
            inasm = False
            continue
        if not t or t.startswith((".", ";")) or t.endswith(":"):
            continue
        op = t.split()[0]
        ws = int(t.split()[1].rstrip(",")) + 1 if op == "s_nop" else 1
        operands = [o.strip() for o in t[len(op):].split(";")[0].split(",")]
        if inasm:
            if op.startswith("v_mfma"):
                pending.append([_regs(operands[0]), 0])
        else:
            used = set()
            for o in operands:
                if o:
                    used |= _regs(o.split()[0])
            for dest, since in pending:
                if dest & used:
                    found.append((kern, i + 1, since, t))
        for p in pending:
            p[1] += ws
        pending = [p for p in pending if p[1] < NEED]
    return found


def late_operands(asm_text):
    """(kernel, line, wait states, instruction) for inline-asm MFMAs that read an A or B operand a
    compiler-emitted VALU instruction wrote fewer than 2 wait states before (the asm's own s_nop
    counts)."""
    found = []
    kern, inasm, recent = None, False, []  # recent: [regs written, wait states since]
    for i, line in enumerate(asm_text.split("\n")):
        t = line.strip()
        m = re.match(r"^(_Z\w+):", t)
        if m:
            kern, recent = m.group(1), []
            continue
        if t.startswith(";;#ASMSTART"):
            inasm = True
            continue
        if t.startswith(";;#ASMEND"):
            inasm = False
            continue
        if not t or t.startswith((".", ";")) or t.endswith(":"):
            continue
        op = t.split()[0]
        ws = int(t.split()[1].rstrip(",")) + 1 if op == "s_nop" else 1
        operands = [o.strip() for o in t[len(op):].split(";")[0].split(",")]
        if inasm and op.startswith("v_mfma"):
            srcs = _regs(operands[1]) | _regs(operands[2])
            for regs, since in recent:
                if since < 2 and regs & srcs:
                    found.append((kern, i + 1, since, t))
        for r in recent:
            r[1] += ws
        recent = [r for r in recent if r[1] < 2]
        if not inasm and op.startswith("v_") and not op.startswith("v_mfma") and operands[0]:
            recent.append([_regs(operands[0].split()[0]), 0])
    return found


def test_scan_finds_planted_late_operand():
    asm = "\n".join([
        "_Zkernel:",
        "\tv_cvt_pk_bf16_f32 v25, v1, v2",
        "\t;;#ASMSTART",
        "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[20:23], v[24:27], a[0:15]",
        "\t;;#ASMEND",
    ])
    assert [(f[0], f[2]) for f in late_operands(asm)] == [("_Zkernel", 0)]
    assert late_operands(asm.replace("\t;;#ASMSTART\n", "\t;;#ASMSTART\n\ts_nop 1\n")) == []


def test_scan_finds_planted_copy():
    asm = "\n".join([
        "_Zkernel:",
        "\t;;#ASMSTART",
        "\ts_nop 1",
        "\tv_mfma_f32_32x32x16_bf16 v[2:17], v[20:23], v[24:27], v[2:17]",
        "\t;;#ASMEND",
        "\tv_add_f32_e32 v30, v31, v32",
        "\tv_mov_b64_e32 v[40:41], v[16:17]",
    ])
    found = early_touches(asm)
    assert [(f[0], f[2]) for f in found] == [("_Zkernel", 2)]
    # after a drain the same copy is clean
    drained = asm.replace("\tv_add_f32_e32", "\t;;#ASMSTART\n\ts_nop 7\n\ts_nop 7\n\ts_nop 3\n\t;;#ASMEND\n"
                                               "\tv_add_f32_e32")
    assert early_touches(drained) == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_no_early_reads_of_asm_mfma_results(tmp_path):
    sys.path.insert(0, os.path.join(ROOT, "pallas-flexattn_amd"))
    import build as b
    b.write_rtc_sources()
    outs, _ = b.compile_units(["--cuda-device-only", "-S"], suffix=".s", out_dir=str(tmp_path))
    text = "\n".join(open(o).read() for o in outs)
    assert ";;#ASMSTART" in text and "v_mfma" in text
    found = early_touches(text)
    assert not found, "\n".join(f"{k} line {ln}: {ws} wait states: {ins}" for k, ln, ws, ins in found[:20])
    # every inline-asm block that writes M0 hands the compiler's value back
    m0 = m0_unrestored(text)
    assert not m0, "inline asm leaves M0 changed: " + "; ".join(m0[:10])
    sg = sgpr_vmem_hazards(text)
    assert not sg, "\n".join(f"line {ln}: {ws} wait states: {ins}" for ln, ws, ins in sg[:20])
    late = late_operands(text)
    assert not late, "\n".join(f"{k} line {ln}: {ws} wait states: {ins}" for k, ln, ws, ins in late[:20])


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_user_mod_kernels_pass_the_same_scans(tmp_path):
    """The kernels compiled at run time for user mods are the same templates with a
    generated policy (user mask on partial tiles, user score with its derivative, tensor
    reads); compiled here with the library's compiler and flags, as the run-time compile
    does, they must pass the same scans."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "pallas-flexattn_amd"))
    import build as b
    from pallas_flexattn import lowering as L
    bias = torch.randn(4, 64)
    mods = L.UserMods(L.lower_mask(lambda q, kv: (kv < 64) | ((q >= kv) & ((q - kv) % 3 != 1))),
                      L.lower_score(lambda s, bb, h, q, kv: 20.0 * torch.tanh((s + bias[h, kv % 64]) / 20.0)))
    src = tmp_path / "user_mods.hip"
    inst = "\n".join(f"template __global__ void fa::{k}<128, 64, 4, true, UserMod>(fa::{a});"
                     for k, a in (("fwd_bf16_kernel", "FwdArgs"), ("dq_bf16_kernel", "BwdArgs"),
                                  ("dkdv_bf16_kernel", "BwdArgs")))
    csrc = os.path.join(ROOT, "pallas-flexattn_amd", "csrc")
    src.write_text(f'#include "fwd_bf16.h"\n#include "bwd_bf16.h"\n{mods.source}\n{inst}\n')
    flags = [f for f in b.FLAGS if f not in ("-shared", "-fPIC")]
    out = tmp_path / "user_mods.s"
    res = subprocess.run([b.HIPCC, *flags, "-I" + csrc, "--cuda-device-only", "-S", str(src), "-o", str(out)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    text = out.read_text()
    assert text.count("v_mfma") > 100
    for name, found in (("early", early_touches(text)), ("late", late_operands(text))):
        assert not found, name + "\n" + "\n".join(f"{k} line {ln}: {ws}: {ins}" for k, ln, ws, ins in found[:20])
    assert not m0_unrestored(text)
    assert not sgpr_vmem_hazards(text)


def _sgprs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def sgpr_vmem_hazards(asm_text, need=5):
    """(line, wait states, instructions) for inline-asm LDS-DMA copies (`buffer_load_* ... lds`)
    whose descriptor SGPRs a VALU instruction wrote fewer than `need` wait states before.  The
    walk goes back from the copy over every path that reaches it: at a label it continues into
    the fall-through predecessor (unless that ends in an unconditional branch) and into every
    branch to the label."""
    lines = [l.strip() for l in asm_text.split("\n")]
    labels, branches_to = {}, {}
    for k, t in enumerate(lines):
        if re.match(r"^[.\w$]+:", t) and not t.startswith(";"):
            labels[t.split(":")[0]] = k
        m = re.match(r"^s_c?branch\w*\s+(\S+)", t)
        if m:
            branches_to.setdefault(m.group(1), []).append(k)

    def is_instr(t):
        return t and not t.startswith(";") and not t.startswith(".") and not re.match(r"^[\w$]+:", t)

    def walk(j, ws, regs, seen):
        """hazards on the paths that end just before line j with ws wait states so far"""
        found = []
        while j >= 0 and ws < need:
            t = lines[j]
            if re.match(r"^[.\w$]+:", t) and not t.startswith(";"):
                name = t.split(":")[0]
                for b in branches_to.get(name, []):
                    if (b, ws) not in seen:
                        seen.add((b, ws))
                        found += walk(b, ws, regs, seen)
                k = j - 1  # fall-through predecessor: the last instruction before the label
                while k >= 0 and not is_instr(lines[k]) and not re.match(r"^[.\w$]+:", lines[k]):
                    k -= 1
                if k < 0 or lines[k].startswith(("s_branch", "s_endpgm", "s_setpc")):
                    return found
                j -= 1
                continue
            j -= 1
            if not is_instr(t):
                continue
            op = t.split()[0]
            if op.startswith("v_") and len(t.split()) > 1 and _sgprs(t.split(None, 1)[1].split(",")[0]) & regs:
                return found + [(ws, t)]
            ws += int(t.split()[1]) + 1 if op == "s_nop" else 1
        return found

    out, in_asm = [], False
    for i, t in enumerate(lines):
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not (in_asm and t.startswith("buffer_load") and t.endswith(" lds")):
            continue
        regs = _sgprs(t.split(None, 1)[1].split(",")[1].strip())
        for ws, u in walk(i - 1, 0, regs, set()):
            out.append((i + 1, ws, u + "  ->  " + t))
    return out


def test_sgpr_vmem_scan_finds_planted_case():
    good = ("\tv_readfirstlane_b32 s12, v48\n\ts_mov_b32 m0, s9\n\t;;#ASMSTART\n\ts_nop 4\n"
            "\tbuffer_load_dwordx4 v192, s[12:15], 0 offen lds\n\t;;#ASMEND\n")
    assert sgpr_vmem_hazards(good) == []
    bad = good.replace("s_nop 4", "s_nop 1")
    found = sgpr_vmem_hazards(bad)
    assert [(ws, ins.split()[1]) for _, ws, ins in found] == [(3, "s12,")]
    # a write of an SGPR the copy does not read is no hazard
    assert sgpr_vmem_hazards(bad.replace("s12, v48", "s20, v48")) == []
    # across a label: found through a branch to it (the write sits before the branch), and
    # through the fall-through edge; not through a fall-through edge cut by s_branch
    tail = bad.split("\n", 1)[1]
    via_branch = "\tv_readfirstlane_b32 s13, v1\n\ts_cbranch_scc1 .LBB0_3\n\ts_nop 7\n\ts_branch .LBB0_9\n.LBB0_3:\n" + tail
    assert [ws for _, ws, _ in sgpr_vmem_hazards(via_branch)] == [4]
    fall = "\tv_readfirstlane_b32 s13, v1\n.LBB0_3:\n" + tail
    assert [ws for _, ws, _ in sgpr_vmem_hazards(fall)] == [3]
    cut = "\tv_readfirstlane_b32 s13, v1\n\ts_branch .LBB0_9\n.LBB0_3:\n" + tail
    assert sgpr_vmem_hazards(cut) == []


def m0_unrestored(asm_text):
    """Inline-asm blocks (their first line) that write M0 without first copying it to an SGPR
    and ending with that SGPR copied back."""
    out, block = [], None
    for line in asm_text.split("\n"):
        t = line.strip().split(";;")[0].strip() if not line.strip().startswith(";;") else line.strip()
        if t.startswith(";;#ASMSTART"):
            block = []
        elif t.startswith(";;#ASMEND"):
            saved, last_write, ok = None, None, True
            for ins in block:
                m = re.match(r"s_mov_b32\s+(s\d+),\s*m0$", ins)
                if m and saved is None and last_write is None:
                    saved = m.group(1)
                    continue
                m = re.match(r"s_mov_b32\s+m0,\s*(\S+)$", ins)
                if m:
                    last_write = m.group(1)
                elif re.search(r"^\S+\s+m0\b", ins):  # any other instruction writing M0
                    last_write = "?"
            if last_write is not None and (saved is None or last_write != saved):
                out.append(block[0] if block else "")
            block = None
        elif block is not None and t:
            block.append(t)
    return out


def test_m0_scan_finds_planted_case():
    good = "\t;;#ASMSTART\n\ts_mov_b32 s9, m0\n\ts_mov_b32 m0, s4\n\tbuffer_load_dwordx4 v1, s[0:3], 0 offen lds\n" \
           "\ts_mov_b32 m0, s9\n\t;;#ASMEND\n"
    bad = "\t;;#ASMSTART\n\ts_mov_b32 m0, s4\n\tbuffer_load_dwordx4 v1, s[0:3], 0 offen lds\n\t;;#ASMEND\n"
    assert m0_unrestored(good) == []
    assert m0_unrestored(bad) == ["s_mov_b32 m0, s4"]
