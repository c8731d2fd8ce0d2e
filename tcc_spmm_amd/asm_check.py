"""Build-time check of the SpMM kernels' gfx950 assembly.

On gfx950 a VALU, memory or LDS instruction that reads a VGPR written by an MFMA is not interlocked:
the compiler must separate them by wait states (16-pass MFMAs such as v_mfma_f32_32x32x8_f16 need
18, which the compiler itself pads to). Kernel variants built during development showed ROCm 7.2's
compiler issuing such reads 2 to 8 wait states after the MFMA, always next to register-spill code
at a loop exit; the variant that did so produced wrong results. The build therefore refuses a kernel
that spills to scratch or reads an MFMA result within REQUIRED wait states on any control-flow path.

check(asm_text) returns a list of problems (empty when the kernels are clean).
"""
from __future__ import annotations

import re

REQUIRED = 18


def _regs(tok: str) -> set:
    """Vector registers an operand names: v7, v[4:7], a[0:15]."""
    out = set()
    for m in re.finditer(r"\b([va])\[(\d+):(\d+)\]", tok):
        out |= {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    for m in re.finditer(r"(?<![\w\[:])([va])(\d+)\b", tok):
        out.add((m.group(1), int(m.group(2))))
    return out


def _operands(rest: str) -> list:
    ops, depth, cur = [], 0, ""
    for ch in rest:
        depth += (ch == "[") - (ch == "]")
        if ch == "," and depth == 0:
            ops.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        ops.append(cur.strip())
    return ops


_PREFIXES = ("v_", "s_", "buffer_", "global_", "ds_", "flat_", "scratch_")
_WRITE_FIRST = ("v_", "global_load", "buffer_load", "ds_read", "ds_load", "scratch_load",
                "ds_bpermute", "ds_permute")


def _parse(lines):
    instrs, labels = [], {}
    for line in lines:
        s = line.split(";")[0].strip()
        m = re.match(r"^(\.LBB\S+):", s)
        if m:
            labels[m.group(1)] = len(instrs)
            continue
        if s.startswith(_PREFIXES):
            instrs.append(s)
    return instrs, labels


def _info(ins: str):
    op, _, rest = ins.partition(" ")
    ops = _operands(rest)
    if op.startswith(_WRITE_FIRST) and ops:
        writes = _regs(ops[0])
        reads = set().union(*[_regs(o) for o in ops[1:]]) if len(ops) > 1 else set()
    elif op.startswith(_PREFIXES[2:]):
        writes, reads = set(), set().union(*[_regs(o) for o in ops]) if ops else set()
    else:
        writes, reads = set(), set()
    return op, writes, reads, ops


def _successors(instrs, labels, i):
    op = instrs[i].split()[0]
    m = re.search(r"(\.LBB\S+)", instrs[i])
    if op.startswith("s_cbranch") and m:
        return [labels[m.group(1)], i + 1]
    if op == "s_branch" and m:
        return [labels[m.group(1)]]
    if op == "s_endpgm" or op.startswith("s_setpc"):
        return []
    return [i + 1]


def _kernel_hazards(instrs, labels):
    infos = [_info(x) for x in instrs]
    found = []
    for i, (op, w, _, _) in enumerate(infos):
        if not op.startswith("v_mfma") or not w:
            continue
        stack = [(j, 0, frozenset(w)) for j in _successors(instrs, labels, i)]
        seen = {}
        while stack:
            j, waits, pending = stack.pop()
            if j >= len(instrs) or waits >= REQUIRED or not pending:
                continue
            if seen.get((j, pending), 1 << 30) <= waits:
                continue
            seen[(j, pending)] = waits
            op2, w2, r2, ops2 = infos[j]
            if op2.startswith("v_mfma"):
                # A dependent MFMA reading the result as its accumulator is interlocked; as a
                # multiplicand it is not.
                hit = (_regs(ops2[1]) | _regs(ops2[2])) & pending if len(ops2) > 2 else set()
            else:
                hit = r2 & pending
            if hit:
                found.append((waits, instrs[i], instrs[j]))
                continue
            if not op2.startswith("v_mfma"):
                pending = pending - w2
            cost = int(instrs[j].split()[1], 0) + 1 if op2 == "s_nop" else 1
            stack.extend((s, waits + cost, pending) for s in _successors(instrs, labels, j))
    return found


def check(asm_text: str) -> list:
    """Problems in every kernel of a gfx950 assembly listing (hipcc --cuda-device-only -S)."""
    lines = asm_text.split("\n")
    problems = []
    starts = [k for k, l in enumerate(lines) if re.match(r"^_Z\S+:", l) and "Kernel" in l]
    for k in starts:
        name = lines[k].split(":")[0]
        end = next((j for j in range(k, len(lines)) if lines[j].startswith(".Lfunc_end")), len(lines))
        body = lines[k + 1:end]
        if any(l.strip().startswith(("scratch_store", "scratch_load", "buffer_store_dword off"))
               for l in body):
            problems.append(f"{name}: spills to scratch")
        instrs, labels = _parse(body)
        for waits, mfma, reader in _kernel_hazards(instrs, labels):
            problems.append(f"{name}: MFMA result read {waits} wait states after `{mfma}` by "
                            f"`{reader}` (needs {REQUIRED})")
    for m in re.finditer(r"\.name:\s+(\S+)\n(?:.*\n){0,40}?\s+\.vgpr_spill_count:\s+(\d+)",
                         asm_text):
        if int(m.group(2)):
            problems.append(f"{m.group(1)}: {m.group(2)} VGPR spills")
    if not starts:
        problems.append("no kernels found in the assembly")
    return problems
