"""Path analysis of gfx950 assembly (test helper): inline-asm vector loads whose destination registers the
compiler does not know to be in flight must not be touched before an s_waitcnt vmcnt(N) that has at least N
vector-memory instructions issued after the load, on every path: around the innermost loop's back-edge and out
of it (the asm is a function's instruction list; backward branches mark loops)."""
import re

_VMEM = re.compile(r"(global_load|global_store|scratch_|buffer_|global_atomic)")


def _regs(text):
    out = set()
    for m in re.finditer(r"v\[(\d+):(\d+)\]", text):
        out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"(?<![\[:\w])v(\d+)(?![\d:\]])", text):
        out.add(int(m.group(1)))
    return out


def function_lines(asm: str, symbol: str):
    """(instruction, inside inline asm) pairs of one function's body."""
    start = asm.index(symbol + ":")
    end = asm.index(".Lfunc_end", start)
    out, in_asm = [], False
    for line in asm[start:end].split("\n"):
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
        elif t.startswith(";;#ASMEND"):
            in_asm = False
        elif t and not t.startswith(";"):
            out.append((t, in_asm))
    return out


def unsafe_asm_loads(ins, opcode="global_load_dwordx4"):
    """[(load, reason)] for inline-asm loads of `opcode` touched before they are known complete; also returns
    how many such loads were checked."""
    labels = {t.split(":")[0]: i for i, (t, _) in enumerate(ins) if t.startswith(".LBB")}
    loops = []
    for i, (t, _) in enumerate(ins):
        m = re.match(r"s_(?:cbranch_\w+|branch)\s+(\.LBB\S+)", t)
        if m and labels.get(m.group(1), len(ins)) < i:
            loops.append((labels[m.group(1)], i))

    def scan(order, dst):
        after = 0
        for j in order:
            t, _ = ins[j]
            if t.startswith(".LBB"):
                continue
            if t.startswith("s_waitcnt") and "vmcnt" in t:
                m = re.search(r"vmcnt\((\d+)\)", t)
                if m and after >= int(m.group(1)):
                    return None
                continue
            if _VMEM.match(t):
                after += 1
            if t.startswith("s_"):
                continue
            parts = t.split(None, 1)
            if len(parts) > 1 and _regs(parts[1]) & dst:
                return f"touched at {j}: {t}"
        return None

    bad, n = [], 0
    for i, (t, in_asm) in enumerate(ins):
        if not (in_asm and t.startswith(opcode + " ")):
            continue
        n += 1
        dst = _regs(t.split(",")[0].split(None, 1)[1])
        inner = [lp for lp in loops if lp[0] <= i <= lp[1]]
        paths = [list(range(i + 1, len(ins)))]
        if inner:
            h, b = min(inner, key=lambda x: x[1] - x[0])
            paths.append(list(range(i + 1, b + 1)) + list(range(h, i + 1)))
        for pth in paths:
            r = scan(pth, dst)
            if r:
                bad.append((t, r))
    return bad, n
