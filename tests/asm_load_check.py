"""Checker for inline-asm vector loads into VGPRs (test infrastructure, CPU only).

The compiler does not see a load written in inline asm: it takes the asm's output register as
written when the asm statement issues, while the hardware writes it when the data returns. If
the compiler reads that register (a copy, a spill, a live-range split) or gives it to another
value before an `s_waitcnt vmcnt(N)` has covered the load, the program reads or loses a value
that has not arrived, or the late return overwrites a register now holding something else.

`check_asm(text)` parses the device assembly of a file (hipcc --offload-device-only -S), and for
every kernel runs a forward dataflow over its basic blocks:

- state: the asm loads that may still be in flight, each with the least number of vector memory
  instructions issued after it on any path (loads, stores and LDS-DMA all count in vmcnt, and
  on gfx9 they complete in issue order);
- `s_waitcnt vmcnt(N)` retires every load with at least N instructions issued after it; 64 or
  more later instructions also retire it (vmcnt is a 6-bit counter, so issue stalls first);
- any instruction that names a register of a load still in flight is a violation, and so is a
  branch whose target is not a label of the same function (the check cannot follow it).

Paths merge by union, keeping the smaller count, so a load counts as retired only when it is
retired on every path.
"""

import re

_VMEM = re.compile(r"^(global|buffer|flat|scratch)_(load|store|atomic)")
_LOAD_DST = re.compile(r"^(global|buffer|flat|scratch)_load_\w+$")
_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_LABEL = re.compile(r"^([.\w$]+):")
_VMCNT_CAP = 64


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


class Instr:
    __slots__ = ("line", "op", "args", "in_asm")

    def __init__(self, line, op, args, in_asm):
        self.line = line
        self.op = op
        self.args = args
        self.in_asm = in_asm


def _parse_function(lines, start):
    """Instructions and labels of the function whose symbol line is `start`, up to .Lfunc_end."""
    instrs, labels = [], {}
    in_asm = False
    for i in range(start + 1, len(lines)):
        raw = lines[i]
        if raw.startswith(".Lfunc_end"):
            break
        if ";;#ASMSTART" in raw:
            in_asm = True
            continue
        if ";;#ASMEND" in raw:
            in_asm = False
            continue
        text = raw.split(";")[0].strip()
        if not text:
            continue
        m = _LABEL.match(text)
        if m:
            labels[m.group(1)] = len(instrs)
            text = text[m.end():].strip()
            if not text:
                continue
        if text.startswith("."):
            continue  # assembler directive
        parts = text.split(None, 1)
        instrs.append(Instr(i + 1, parts[0], parts[1] if len(parts) > 1 else "", in_asm))
    return instrs, labels


def _blocks(instrs, labels):
    """Basic blocks as (first, last) index pairs and their successor block numbers."""
    starts = {0} | set(labels.values())
    for j, ins in enumerate(instrs):
        if ins.op.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc", "s_swappc")):
            starts.add(j + 1)
    starts = sorted(s for s in starts if s < len(instrs))
    index = {s: b for b, s in enumerate(starts)}
    blocks, succs = [], []
    for b, s in enumerate(starts):
        e = (starts[b + 1] if b + 1 < len(starts) else len(instrs)) - 1
        blocks.append((s, e))
        last = instrs[e]
        nxt = [b + 1] if b + 1 < len(starts) else []
        if last.op == "s_endpgm":
            succs.append([])
        elif last.op.startswith(("s_setpc", "s_swappc")):
            succs.append(None)  # indirect: cannot be followed
        elif last.op == "s_branch" or last.op.startswith("s_cbranch"):
            target = last.args.split(",")[0].strip()
            if target not in labels:
                succs.append(None)
            else:
                tgt = [index[labels[target]]]
                succs.append(tgt if last.op == "s_branch" else sorted(set(tgt + nxt)))
        else:
            succs.append(nxt)
    return blocks, succs


def _vmcnt(ins):
    if ins.op != "s_waitcnt":
        return None
    m = re.search(r"vmcnt\((\d+)\)", ins.args)
    if m:
        return int(m.group(1))
    if ins.args.strip() == "0":
        return 0
    return None


def _is_asm_vgpr_load(ins):
    if not ins.in_asm or not _LOAD_DST.match(ins.op) or "_lds" in ins.op:
        return False
    return not re.search(r"\blds\b", ins.args)


def check_function(instrs, labels):
    """Violations of one function: (load line, offending line, offending text)."""
    if not instrs:
        return []
    blocks, succs = _blocks(instrs, labels)
    dst = {}
    for ins in instrs:
        if _is_asm_vgpr_load(ins):
            dst[ins.line] = _regs(ins.args.split(",")[0])
    violations = set()
    if not dst:
        return []
    state_in = [None] * len(blocks)
    state_in[0] = {}
    work = [0]
    while work:
        b = work.pop()
        state = dict(state_in[b])
        s, e = blocks[b]
        for j in range(s, e + 1):
            ins = instrs[j]
            n = _vmcnt(ins)
            if n is not None:
                state = {ld: c for ld, c in state.items() if c < n}
            names = _regs(ins.args)
            for ld in state:
                if names & dst[ld]:
                    violations.add((ld, ins.line, (ins.op + " " + ins.args).strip()))
            if _VMEM.match(ins.op):
                state = {ld: c + 1 for ld, c in state.items() if c + 1 < _VMCNT_CAP}
            if ins.line in dst:
                state[ins.line] = 0
        if succs[b] is None:
            if state:
                violations.add((min(state), instrs[e].line, "branch the check cannot follow"))
            continue
        for t in succs[b]:
            old = state_in[t]
            if old is None:
                new = dict(state)
            else:
                new = dict(old)
                for ld, c in state.items():
                    new[ld] = min(c, new[ld]) if ld in new else c
            if new != old:
                state_in[t] = new
                work.append(t)
    return sorted(violations)


def check_asm(text):
    """{kernel symbol: [violations]} for every function of an assembly listing, and the number
    of inline-asm VGPR loads seen."""
    lines = text.split("\n")
    result, nloads = {}, 0
    for i, raw in enumerate(lines):
        m = re.match(r"^(_Z\w+):", raw)
        if not m:
            continue
        instrs, labels = _parse_function(lines, i)
        nloads += sum(1 for ins in instrs if _is_asm_vgpr_load(ins))
        result[m.group(1)] = check_function(instrs, labels)
    return result, nloads
