"""In-flight register check for kernels that issue global loads from inline asm.

A register written by a global load issued from an inline-asm statement is
in flight until an ``s_waitcnt vmcnt(k)`` retires it, which happens once at
least k vector-memory instructions have been issued after the load (vmcnt
retires loads and stores in issue order). The compiler believes the asm
statement wrote the register when the statement ended, so it is free to copy,
spill or reuse that register before the wait; a copy taken there reads the
old contents. (A copy of this kind, placed in front of one branch's wait,
once made a kernel compute with a stale Q operand.)

``check_listing`` parses a device assembly listing (``hipcc -S
--cuda-device-only``), builds each function's control-flow graph and
propagates the set of in-flight registers along it, with the number of
vector-memory instructions issued since each one's load (the minimum over
the paths that reach a point). Any instruction other than a wait that names
an in-flight register is reported, except as the destination of another
load: loads write their registers in issue order, so the younger load's
value is the one that stays (its address operands are still checked).
Direct-to-LDS loads (``... lds``) write no register and are only counted.
"""
from __future__ import annotations

import re
from dataclasses import dataclass

_VMEM = re.compile(r"^(buffer|global|flat|scratch)_")
_VMEM_LOAD = re.compile(r"^(buffer|global|flat)_load_")
_REG_RANGE = re.compile(r"\b([va])\[(\d+):(\d+)\]")
_REG_ONE = re.compile(r"\b([va])(\d+)\b")
_LABEL = re.compile(r"^(\.?[A-Za-z_$][\w.$]*):")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")
_CAP = 64


@dataclass
class Violation:
    function: str
    line: int          # 1-based line in the listing
    text: str
    registers: list

    def __str__(self) -> str:
        regs = ", ".join(self.registers)
        return f"{self.function}: line {self.line}: `{self.text}` names in-flight {regs}"


def _regs(operands: str) -> set:
    out = set()
    for kind, lo, hi in _REG_RANGE.findall(operands):
        out.update(f"{kind}{i}" for i in range(int(lo), int(hi) + 1))
    rest = _REG_RANGE.sub(" ", operands)
    out.update(f"{kind}{i}" for kind, i in _REG_ONE.findall(rest))
    return out


def _vmcnt(mnemonic: str, operands: str):
    """The vmcnt limit of an s_waitcnt, or None when it does not wait on vmcnt."""
    if mnemonic != "s_waitcnt":
        return None
    m = _VMCNT.search(operands)
    if m:
        return int(m.group(1))
    ops = operands.strip()
    if re.fullmatch(r"(0x[0-9a-fA-F]+|\d+)", ops):
        v = int(ops, 0)
        return (v & 0xF) | ((v >> 14) & 0x3) << 4
    return None


@dataclass
class _Inst:
    line: int
    text: str
    mnemonic: str
    operands: str
    in_asm: bool


def _functions(text: str):
    """{name: [label or _Inst, ...]} for every function body in the listing."""
    funcs, cur, name, in_asm = {}, None, None, False
    for no, raw in enumerate(text.splitlines(), 1):
        line = raw.rstrip()
        s = line.strip()
        if cur is None:
            m = _LABEL.match(line)
            if m and not line.startswith((" ", "\t")) and not m.group(1).startswith(".L"):
                name, cur = m.group(1), []
            continue
        if s.startswith(".Lfunc_end"):
            funcs[name] = cur
            cur, name, in_asm = None, None, False
            continue
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith(";") or s.startswith("//"):
            continue
        m = _LABEL.match(s)
        if m and not line.startswith((" ", "\t")):
            cur.append(m.group(1))
            continue
        if s.startswith("."):
            continue
        body = s.split(";", 1)[0].strip()
        if not body:
            continue
        parts = body.split(None, 1)
        cur.append(_Inst(no, body, parts[0], parts[1] if len(parts) > 1 else "", in_asm))
    return funcs


def _blocks(items):
    """Basic blocks [(label, [insts], [successor labels])]."""
    blocks, label, insts = [], "<entry>", []

    def close(nxt_label):
        nonlocal label, insts
        blocks.append([label, insts, None])
        label, insts = nxt_label, []

    n = 0
    for it in items:
        if isinstance(it, str):
            if insts or label != "<entry>" or blocks:
                close(it)
            else:
                label = it
            continue
        insts.append(it)
        if it.mnemonic.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc", "s_trap")):
            n += 1
            close(f"<fall{n}>")
    blocks.append([label, insts, None])
    index = {b[0]: i for i, b in enumerate(blocks)}
    for i, b in enumerate(blocks):
        last = b[1][-1] if b[1] else None
        nxt = [blocks[i + 1][0]] if i + 1 < len(blocks) else []
        if last is None:
            b[2] = nxt
        elif last.mnemonic == "s_branch":
            b[2] = [last.operands.split()[0]]
        elif last.mnemonic.startswith("s_cbranch"):
            b[2] = [last.operands.split()[0]] + nxt
        elif last.mnemonic.startswith(("s_endpgm", "s_setpc", "s_trap")):
            b[2] = []
        else:
            b[2] = nxt
        b[2] = [s for s in b[2] if s in index]
    return blocks, index


def _transfer(insts, state, function, report):
    """Run one block over `state` ({register: vector-memory ops since its load});
    returns the exit state; appends violations to `report` when given."""
    st = dict(state)
    for inst in insts:
        limit = _vmcnt(inst.mnemonic, inst.operands)
        if limit is not None:
            st = {r: c for r, c in st.items() if c < limit}
            continue
        is_vmem = bool(_VMEM.match(inst.mnemonic))
        named = _regs(inst.operands)
        writes = set()
        reg_load = is_vmem and bool(_VMEM_LOAD.match(inst.mnemonic)) and " lds" not in f" {inst.operands} "
        if reg_load:
            # A load's destination may be a register still in flight from an
            # older load: loads retire, and write their registers, in issue
            # order, so the younger value lands last. Its address operands
            # are still checked.
            dest = _regs(inst.operands.split(",", 1)[0])
            named = named - dest
            if inst.in_asm:
                writes = dest
        hit = sorted((named & st.keys()), key=lambda r: (r[0], int(r[1:])))
        if hit and report is not None:
            report.append(Violation(function, inst.line, inst.text, hit))
        if is_vmem:
            st = {r: min(c + 1, _CAP) for r, c in st.items()}
        for r in writes:
            st[r] = 0
    return st


def _merge(a, b):
    out = dict(a)
    for r, c in b.items():
        out[r] = min(out[r], c) if r in out else c
    return out


def check_function(name, items):
    blocks, index = _blocks(items)
    entry = [None] * len(blocks)
    entry[0] = {}
    work = [0]
    while work:
        i = work.pop()
        out = _transfer(blocks[i][1], entry[i], name, None)
        for s in blocks[i][2]:
            j = index[s]
            new = out if entry[j] is None else _merge(entry[j], out)
            if new != entry[j]:
                entry[j] = new
                work.append(j)
    report = []
    for i, b in enumerate(blocks):
        if entry[i] is not None:
            _transfer(b[1], entry[i], name, report)
    return report


def check_listing(text: str, only=None):
    """Violations in every function of an assembly listing (or those whose
    name contains one of `only`)."""
    out = []
    for name, items in _functions(text).items():
        if only and not any(o in name for o in only):
            continue
        out.extend(check_function(name, items))
    return out


def count_asm_loads(text: str) -> int:
    """Register-writing global loads issued from inline asm in the listing."""
    n = 0
    for items in _functions(text).values():
        for it in items:
            if isinstance(it, _Inst) and it.in_asm and _VMEM_LOAD.match(it.mnemonic) and " lds" not in f" {it.operands} ":
                n += 1
    return n


if __name__ == "__main__":
    import sys
    for path in sys.argv[1:]:
        txt = open(path).read()
        v = check_listing(txt)
        print(f"{path}: {count_asm_loads(txt)} register-writing asm loads, {len(v)} violations")
        for x in v[:20]:
            print("  ", x)
