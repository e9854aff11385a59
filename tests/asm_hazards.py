"""Scanner for one class of gfx950 code-generation hazard in this library's
own AMD assembly: a non-MFMA instruction that reads or writes the destination
registers of a v_mfma_* fewer than W wait states after it, along any control
flow path (straight line or through branches).

Such a read was once produced for the prefill kernel (a branch between an
MFMA and the use of its result let an AGPR read land one instruction after
the MFMA; the scores came out wrong for fp32 pools with G = 1).  The test
compiles every source that issues MFMAs to assembly (hipcc -S, device code
only) and requires zero findings.

Usage as a script: python tests/asm_hazards.py file.s [W]
"""
from __future__ import annotations

import re
import sys

_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)(?!\w))")


def regs(text: str) -> set:
    """VGPR / AGPR indices named in an operand string, as (kind, index)."""
    out = set()
    for m in _REG.finditer(text):
        k = m.group(1)
        if m.group(4) is not None:
            out.add((k, int(m.group(4))))
        else:
            out.update((k, i) for i in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def functions(lines):
    """(name, body lines) of every kernel / function in an assembly listing."""
    cur, name = None, None
    for ln in lines:
        m = re.match(r"^(_Z\S+):", ln)
        if m:
            if cur is not None:
                yield name, cur
            name, cur = m.group(1), []
            continue
        if cur is not None:
            if ln.startswith("\t.end_amdgpu") or re.match(r"^\.Lfunc_end", ln):
                yield name, cur
                cur = None
                continue
            cur.append(ln)


def _wait_states(ins: str) -> int:
    parts = ins.split()
    if parts[0] == "s_nop":
        return int(parts[1], 0) + 1
    return 1


def analyse(body, window: int = 8):
    """Findings (use index, mfma index, wait states between, use, mfma)."""
    ins, labels = [], {}
    for ln in body:
        s = ln.split(";")[0].rstrip()
        if not s.strip():
            continue
        m = re.match(r"^(\.LBB\S+):", s)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        if s.strip().startswith("."):
            continue
        ins.append(s.strip())
    n = len(ins)
    preds = [[] for _ in range(n)]
    for i, t in enumerate(ins):
        op = t.split()[0]
        if op.startswith("s_cbranch") or op == "s_branch":
            tgt = t.split()[-1]
            if tgt in labels and labels[tgt] < n:
                preds[labels[tgt]].append(i)
        if op not in ("s_branch", "s_endpgm", "s_setpc_b64") and i + 1 < n:
            preds[i + 1].append(i)
    bad = []
    for i, t in enumerate(ins):
        if "mfma" in t.split()[0]:
            continue
        touched = regs(t)
        if not touched:
            continue
        stack = [(p, 0) for p in preds[i]]
        seen = {}
        while stack:
            j, d = stack.pop()
            if d >= window or seen.get(j, 1 << 30) <= d:
                continue
            seen[j] = d
            tj = ins[j]
            if "v_mfma" in tj.split()[0]:
                dst = regs(tj.split(None, 1)[1].split(",")[0])
                if dst & touched:
                    bad.append((i, j, d, t, tj))
                    continue
            stack.extend((p, d + _wait_states(tj)) for p in preds[j])
    return bad


def scan(text: str, window: int = 8):
    """All findings of an assembly listing: [(function, wait states, mfma, use)]."""
    out = []
    for name, body in functions(text.split("\n")):
        for _, _, d, use, mfma in analyse(body, window):
            out.append((name, d, mfma, use))
    return out


if __name__ == "__main__":
    w = int(sys.argv[2]) if len(sys.argv) > 2 else 8
    found = scan(open(sys.argv[1]).read(), w)
    for name, d, mfma, use in found[:20]:
        print(f"{name[:60]}: {d} wait states: {mfma[:50]} -> {use[:50]}")
    print("findings", len(found))
    sys.exit(1 if found else 0)
