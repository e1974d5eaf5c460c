"""Scan of gfx950 assembly built here for MFMA results read too early.

The hardware does not interlock a VALU read (or an MFMA A/B operand read) of an MFMA destination:
the program must leave enough wait states between them. Inside a basic block the compiler pads
them itself. This scan takes, for each MFMA opcode, the smallest number of wait states the
compiler leaves before a dependent read inside one block (its own rule for that opcode), then
follows every path through conditional branches and reports dependent reads reached through a
branch with fewer wait states than that rule. An instruction counts one wait state, `s_nop N`
counts N + 1."""

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
