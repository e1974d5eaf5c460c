"""Scans of gfx950 assembly built here for hazards the compiler does not pad.

MFMA results read too early:

The hardware does not interlock a VALU read (or an MFMA A/B operand read) of an MFMA destination:
the program must leave enough wait states between them. Inside a basic block the compiler pads
them itself. This scan takes, for each MFMA opcode, the smallest number of wait states the
compiler leaves before a dependent read inside one block (its own rule for that opcode), then
follows every path through conditional branches and reports dependent reads reached through a
branch with fewer wait states than that rule. An instruction counts one wait state, `s_nop N`
counts N + 1.

Inline asm: the compiler's hazard padding does not look into inline asm statements, so an asm
vector memory instruction whose SGPR base address a VALU instruction (v_readlane restoring a
spilled SGPR, v_readfirstlane) wrote fewer than 5 wait states earlier, on any path, reads a stale
base (AMD's CDNA3 ISA guide, "Manually Inserted Wait States"); likewise an asm VALU instruction
reading the result of a transcendental with no wait state between them (gfx940 and later).
inline_asm_hazards() walks back from every such asm instruction over all predecessors."""

from __future__ import annotations

import re
from pathlib import Path

_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)\b)")


def regs(text: str) -> set[tuple[str, int]]:
    out = set()
    for m in _REG.finditer(text):
        if m.group(4) is not None:
            out.add((m.group(1), int(m.group(4))))
        else:
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def functions(asm: str) -> dict[str, list[str]]:
    """Instructions and branch labels of every kernel in an assembly listing."""
    funcs: dict[str, list[str]] = {}
    current = None
    for line in asm.splitlines():
        s = line.split(";")[0].strip()
        if re.match(r"^_Z\w+:$", s):
            current = s[:-1]
            funcs[current] = []
        elif current is not None and s and (not s.startswith(".") or s.startswith(".LBB")):
            funcs[current].append(s)
    return funcs


def dependent_reads(ins: list[str], i: int, limit: int = 40):
    """(wait states, branch labels taken, instruction) of the first dependent read of MFMA i's
    destination on every path, up to `limit` wait states."""
    dregs = regs(ins[i].split(None, 1)[1].split(",")[0])
    labels = {x[:-1]: k for k, x in enumerate(ins) if x.endswith(":")}
    found, stack, seen = [], [(i + 1, 0, ())], set()
    while stack:
        j, waited, path = stack.pop()
        while j < len(ins) and waited < limit:
            t = ins[j]
            if t.endswith(":"):
                j += 1
                continue
            op, _, operands = t.partition(" ")
            if op.startswith("s_nop"):
                waited += int(operands) + 1
                j += 1
                continue
            if op == "s_endpgm":
                break
            if op.startswith("s_cbranch") or op == "s_branch":
                target = operands.strip()
                if target in labels and (target, waited) not in seen:
                    seen.add((target, waited))
                    stack.append((labels[target] + 1, waited + 1, path + (target,)))
                if op == "s_branch":
                    break
            elif op.startswith("v_mfma"):
                parts = operands.split(",")
                if regs(",".join(parts[1:3])) & dregs:  # A/B operands (C is forwarded)
                    found.append((waited, path, t))
                    break
                if regs(parts[0]) & dregs:
                    break
            elif op.startswith("v_"):
                dst, _, src = operands.partition(",")
                if regs(src) & dregs:
                    found.append((waited, path, t))
                    break
                if regs(dst) & dregs:
                    break
            waited += 1
            j += 1
    return found


def scan(listings: list[str]):
    """(rule per opcode, cross-branch reads, cross-branch reads below the rule)."""
    rule: dict[str, int] = {}
    cross = []
    for asm in listings:
        for name, ins in functions(asm).items():
            for i, line in enumerate(ins):
                op = line.split()[0]
                if not op.startswith("v_mfma"):
                    continue
                for waited, path, t in dependent_reads(ins, i):
                    if path:
                        cross.append((op, waited, name, path, line, t))
                    else:
                        rule[op] = min(rule.get(op, 1 << 30), waited)
    short = [c for c in cross if c[1] < rule.get(c[0], 0)]
    return rule, cross, short


def device_assembly(source: Path, out: Path, extra: tuple[str, ...] = ()) -> str:
    """hipcc's gfx950 assembly of one source, with the library's compile flags."""
    import subprocess

    from tessery_amd import _build

    cmd = [_build.hipcc(), *_build.FLAGS, *_build.SOURCE_FLAGS.get(source.name, ()), *extra,
           "-x", "hip", "-I", str(_build.ROOT / "include"), "-I", str(source.parent),
           "--cuda-device-only", "-S", str(source), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


_SREG = re.compile(r"\bs(?:\[(\d+):(\d+)\]|(\d+)\b)")
_VMEM = ("global_", "buffer_", "scratch_", "flat_")
_TRANS = ("v_rcp_", "v_rsq_", "v_sqrt_", "v_exp_", "v_log_", "v_sin_", "v_cos_", "v_rcp_iflag")


def sregs(text: str) -> set[int]:
    out = set()
    for m in _SREG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def functions_with_asm(asm: str) -> dict[str, list[tuple[str, bool]]]:
    """Instructions (with an inline-asm flag) and branch labels of every kernel."""
    funcs: dict[str, list[tuple[str, bool]]] = {}
    current, inside = None, False
    for line in asm.splitlines():
        raw = line.strip()
        if raw == ";;#ASMSTART":
            inside = True
            continue
        if raw == ";;#ASMEND":
            inside = False
            continue
        s = line.split(";")[0].strip()
        if re.match(r"^_Z\w+:$", s):
            current = s[:-1]
            funcs[current] = []
        elif current is not None and s and (not s.startswith(".") or s.startswith(".LBB")):
            funcs[current].append((s, inside))
    return funcs


def _predecessors(ins: list[tuple[str, bool]]) -> list[list[int]]:
    labels = {t[:-1]: k for k, (t, _) in enumerate(ins) if t.endswith(":")}
    preds: list[list[int]] = [[] for _ in ins]
    for k, (t, _) in enumerate(ins):
        op, _, operands = t.partition(" ")
        if op.startswith("s_cbranch") or op == "s_branch":
            target = operands.strip()
            if target in labels:
                preds[labels[target]].append(k)
        if op not in ("s_branch", "s_endpgm", "s_setpc_b64") and k + 1 < len(ins):
            preds[k + 1].append(k)
    return preds


def _writer_within(ins, preds, i, need, is_writer):
    """Instructions before i, on any path, fewer than `need` wait states back, that is_writer
    accepts: (wait states, instruction)."""
    found, stack, seen = [], [(k, 0) for k in preds[i]], set()
    while stack:
        k, waited = stack.pop()
        if (k, waited) in seen or waited >= need:
            continue
        seen.add((k, waited))
        t = ins[k][0]
        if t.endswith(":"):
            stack.extend((p, waited) for p in preds[k])
            continue
        op, _, operands = t.partition(" ")
        if is_writer(op, operands, ins[k][1]):
            found.append((waited, t))
            continue
        step = int(operands) + 1 if op == "s_nop" else 1
        stack.extend((p, waited + step) for p in preds[k])
    return found


def inline_asm_hazards(listings: list[str]):
    """(kernel, instruction, wait states, writer) for every asm vector memory instruction whose
    SGPR operands a VALU wrote fewer than 5 wait states before, every asm VALU instruction reading
    a transcendental's result with no wait state between, and every MFMA reading a VGPR that an
    asm VALU instruction wrote fewer than 2 wait states before (the compiler pads neither the
    asm's reads nor the reads of what the asm wrote)."""
    out = []
    for asm in listings:
        for name, ins in functions_with_asm(asm).items():
            preds = _predecessors(ins)
            for i, (t, inside) in enumerate(ins):
                op, _, operands = t.partition(" ")
                if not inside:
                    if op.startswith("v_mfma"):
                        msrc = regs(operands.partition(",")[2])

                        def asm_valu_writer(wop, wops, winside, msrc=msrc):
                            return (winside and wop.startswith("v_") and
                                    bool(regs(wops.split(",")[0]) & msrc))

                        for waited, w in _writer_within(ins, preds, i, 2, asm_valu_writer):
                            out.append((name, t, waited, w))
                    continue
                if op.startswith(_VMEM):
                    srcs = sregs(operands)
                    if not srcs:
                        continue

                    def sgpr_writer(wop, wops, _winside, srcs=srcs):
                        if not wop.startswith("v_"):
                            return False
                        return bool(sregs(wops.split(",")[0]) & srcs)

                    for waited, w in _writer_within(ins, preds, i, 5, sgpr_writer):
                        out.append((name, t, waited, w))
                elif op.startswith("v_"):
                    vsrc = regs(operands.partition(",")[2])

                    def trans_writer(wop, wops, _winside, vsrc=vsrc):
                        return wop.startswith(_TRANS) and bool(regs(wops.split(",")[0]) & vsrc)

                    for waited, w in _writer_within(ins, preds, i, 1, trans_writer):
                        out.append((name, t, waited, w))
    return out


def asm_load_reuse(listings: list[str]):
    """(kernel, instruction) for every instruction that reads or writes a VGPR an inline asm
    global load is still filling. The compiler does not know these loads are in flight: each one
    stays pending until a s_waitcnt vmcnt(N) that retires it (vector memory operations retire in
    issue order, so vmcnt(N) retires every one with N or more younger ones). Paths are followed
    through branches; the structurizer's flow flags (s_mov_b64 s[n:n+1], -1 / 0 tested by
    s_and(n2)_b64 vcc, exec, s[n:n+1]) prune the paths they exclude, and exec-zero branches are
    taken as not taken (the asm loads sit in wave-uniform code)."""
    out = []
    for asm in listings:
        for name, ins in functions_with_asm(asm).items():
            labels = {t[:-1]: k for k, (t, _) in enumerate(ins) if t.endswith(":")}
            seen: dict = {}
            work = [(0, (), ())]
            reports = set()
            while work:
                i, pend, consts = work.pop()
                key = (i, consts)
                prev = seen.get(key)
                # pend: ((reg, younger), ...); merge keeps every reg at its fewest younger ops
                merged = dict(prev) if prev else {}
                changed = prev is None
                for r, k in pend:
                    if r not in merged or k < merged[r]:
                        merged[r] = k
                        changed = True
                if not changed:
                    continue
                seen[key] = tuple(sorted(merged.items()))
                p = dict(merged)
                c = dict(consts)
                vcc = c.pop("vcc", None)
                t, inside = ins[i]
                if t.endswith(":"):
                    nxt = [i + 1]
                else:
                    op, _, operands = t.partition(" ")
                    m = re.search(r"vmcnt\((\d+)\)", t) if op == "s_waitcnt" else None
                    if m:
                        n = int(m.group(1))
                        p = {r: k for r, k in p.items() if k < n}
                    elif op.startswith(_VMEM):
                        dst = operands.split(",")[0]
                        vdst = regs(dst) if inside and "load" in op and "lds" not in op else set()
                        touched = regs(operands) & {("v", r) for r in p}
                        if touched:
                            reports.add((name, t))
                        p = {r: k + 1 for r, k in p.items()}
                        for r in vdst:
                            p[r[1]] = 0
                    else:
                        if regs(t) & {("v", r) for r in p}:
                            reports.add((name, t))
                    m = re.match(r"s_mov_b64 s\[(\d+):\d+\], (-1|0)$", t)
                    if m:
                        c[int(m.group(1))] = int(m.group(2))
                    else:
                        for md in re.finditer(r"^s_\w+ s\[(\d+):\d+\]|^s_\w+ s(\d+),", t):
                            reg = int(md.group(1) or md.group(2))
                            c.pop(reg, None)
                            c.pop(reg - 1, None)
                    if re.match(r"s_\w+ vcc|v_\w+_e32 .*vcc|v_cmp", t):
                        vcc = None
                    m = re.match(r"s_andn2_b64 vcc, exec, s\[(\d+):\d+\]$", t)
                    if m and int(m.group(1)) in c:
                        vcc = c[int(m.group(1))] == 0
                    m = re.match(r"s_and_b64 vcc, exec, s\[(\d+):\d+\]$", t)
                    if m and int(m.group(1)) in c:
                        vcc = c[int(m.group(1))] == -1
                    if vcc is not None and not op.startswith("s_cbranch"):
                        c["vcc"] = vcc
                    if op in ("s_endpgm", "s_setpc_b64"):
                        nxt = []
                    elif op == "s_branch":
                        nxt = [labels[operands.strip()]]
                    elif op.startswith("s_cbranch"):
                        target = labels[operands.strip()]
                        if op == "s_cbranch_execz":
                            nxt = [i + 1]
                        elif op == "s_cbranch_execnz":
                            nxt = [target]
                        elif op in ("s_cbranch_vccz", "s_cbranch_vccnz") and vcc is not None:
                            nxt = [target] if (vcc == (op == "s_cbranch_vccnz")) else [i + 1]
                        else:
                            nxt = [target, i + 1]
                    else:
                        nxt = [i + 1]
                ct = tuple(sorted(c.items(), key=lambda kv: str(kv[0])))
                for j in nxt:
                    if j < len(ins):
                        work.append((j, tuple(p.items()), ct))
            out.extend(sorted(reports))
    return out
