"""Build-time check of the GEMM kernels' inline-asm LDS reads (brik_gemm*, gemm.hip).

The multiply loop issues its LDS reads as inline asm (gemm.hip: ds_read_b128 / ds_read_u16, then
lds_wait and tie), so the compiler does not know that their destination registers are written
asynchronously. Correctness then rests on register allocation: no instruction may read or write a
destination register of such a read before an `s_waitcnt lgkmcnt` has retired it.

This script disassembles the built code object (llvm-objdump, our own build) and checks exactly that
on every path through each checked kernel: it builds the kernel's control-flow graph from the branch
instructions (targets from their 16-bit word offsets; a conditional branch also falls through, an
unconditional one and s_endpgm do not) and propagates the registers still pending from an LDS read
forward to a fixed point, so a read issued at the bottom of a loop is still pending at the loop's head
on the back edge. The disassembly does not tell the asm reads from the compiler's own, so every
ds_read_b128 / ds_read_u16 is tracked. A pending register carries its age, the number of LGKM-counted
operations (LDS, scalar memory) issued after its read, and at a join the smaller age of the paths:
LDS operations complete in issue order, so `s_waitcnt lgkmcnt(N)` retires the reads of age N or more,
unless a scalar memory load may be in flight (those complete out of order, and then only lgkmcnt(0)
retires anything). An instruction that touches a pending register is reported.

Usage: python -m brimkern_amd.check_lds_reads <code object>   (exit status 1 on a violation)
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
OBJDUMP = os.path.join(ROCM, "llvm", "bin", "llvm-objdump")
ASM_READS = ("ds_read_b128", "ds_read_u16")
MAX_AGE = 16          # lgkmcnt holds at most 15 on gfx9: an older read is retired by any lgkmcnt wait


def _regs(op: str) -> set:
    m = re.match(r"v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op)
    return {int(m.group(1))} if m else set()


def _checked(fn: str) -> bool:
    """The tiled GEMM kernels (gemm_body): brik_gemm_<fmt>_<tile> and brik_gemmg_q4_<tile>. The split-K
    kernels and the f16-weight LDS-tiled kernel read LDS the ordinary way (compiler-tracked waits)."""
    return fn.startswith(("brik_gemm_", "brik_gemmg_")) and not fn.startswith(("brik_gemm_sk_", "brik_gemm_f16w"))


def _kernels(disasm: str) -> dict:
    """{kernel: [(address or None, instruction text)]} from llvm-objdump -d output (the address is the
    one in the trailing comment)."""
    out, fn = {}, None
    for raw in disasm.split("\n"):
        m = re.match(r"^[0-9a-f]+ <([^>]+)>:", raw)
        if m:
            fn = m.group(1)
            out[fn] = []
            continue
        if fn is None:
            continue
        line = raw.split("//")[0].strip()
        if not line:
            continue
        am = re.search(r"//\s*([0-9A-Fa-f]+):", raw)
        out[fn].append((int(am.group(1), 16) if am else None, line))
    return out


def _successors(code: list) -> list:
    """Successor indices of every instruction (branch targets from the SOPP word offset)."""
    at = {a: i for i, (a, _) in enumerate(code) if a is not None}
    succ = []
    for i, (a, line) in enumerate(code):
        op = line.split(None, 1)[0]
        nxt = [i + 1] if i + 1 < len(code) else []
        if op == "s_endpgm":
            succ.append([])
            continue
        if op == "s_branch" or op.startswith("s_cbranch"):
            tgt = None
            m = re.match(r"\S+\s+(-?\d+)", line)
            if m and a is not None:
                off = int(m.group(1))
                off = off - 65536 if off >= 32768 else off
                tgt = at.get(a + 4 + 4 * off)
            if op == "s_branch":
                succ.append([tgt] if tgt is not None else nxt)
            else:
                succ.append(nxt + ([tgt] if tgt is not None else []))
            continue
        succ.append(nxt)
    return succ


def _lgkm_wait(line: str):
    """N of an s_waitcnt that names lgkmcnt(N), else None."""
    m = re.search(r"lgkmcnt\((\d+)\)", line)
    return int(m.group(1)) if m else None


def _join(a, b):
    """Pending states (frozenset of (register, age), scalar load in flight): union, smaller age."""
    if a is None:
        return b
    ages = dict(a[0])
    for r, g in b[0]:
        ages[r] = min(g, ages.get(r, g))
    return frozenset(ages.items()), a[1] or b[1]


def _step(state, op: str, wait, writes):
    regs, smem = state
    if op == "s_waitcnt" and wait is not None:
        if wait == 0:
            return frozenset(), False
        if smem:
            return regs, smem
        return frozenset((r, g) for r, g in regs if g < wait), smem
    lgkm = op.startswith("ds_") or op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime"))
    if not lgkm:
        return state
    aged = {r: min(g + 1, MAX_AGE) for r, g in regs}
    for r in writes:
        aged[r] = 0
    return frozenset(aged.items()), smem or op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime"))


def _check_kernel(fn: str, code: list) -> list:
    n = len(code)
    succ = _successors(code)
    parsed = []
    for _, line in code:
        parts = line.split(None, 1)
        ops = [o.strip().split()[0] for o in parts[1].split(",") if o.strip()] if len(parts) > 1 else []
        used = set()
        for o in ops:
            used |= _regs(o)
        wait = _lgkm_wait(line) if parts[0] == "s_waitcnt" else None
        writes = _regs(ops[0]) if parts[0] in ASM_READS and ops else set()
        parsed.append((parts[0], used, wait, writes))
    pend_in = [None] * n                       # pending state at entry (None: not reached yet)
    if n:
        pend_in[0] = (frozenset(), False)
    work = [0] if n else []
    while work:
        i = work.pop()
        op, used, wait, writes = parsed[i]
        out = _step(pend_in[i], op, wait, writes)
        for j in succ[i]:
            new = _join(pend_in[j], out)
            if new != pend_in[j]:
                pend_in[j] = new
                work.append(j)
    bad = []
    for i, (op, used, wait, writes) in enumerate(parsed):
        if pend_in[i] is None or op.startswith("ds_read"):
            continue
        hit = used & {r for r, _ in pend_in[i][0]}
        if hit:
            bad.append(f"{fn}: '{code[i][1]}' touches v{sorted(hit)} before the LDS read that writes it has "
                       f"been waited for")
    return bad


def check(disasm: str) -> list:
    """Violations in `disasm` (llvm-objdump -d text) of the kernels _checked selects."""
    out = []
    for fn, code in _kernels(disasm).items():
        if _checked(fn):
            out += _check_kernel(fn, code)
    return out


def check_file(path: str) -> list:
    if not os.path.exists(OBJDUMP):
        raise RuntimeError(f"{OBJDUMP} is missing: the LDS-read register check of the GEMM kernels cannot run "
                           "(set ROCM_PATH to a ROCm install with llvm-objdump)")
    text = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", path], capture_output=True, text=True,
                          check=True).stdout
    return check(text)


if __name__ == "__main__":
    bad = check_file(sys.argv[1])
    for b in bad[:20]:
        print(b)
    print(f"{len(bad)} violation(s)")
    sys.exit(1 if bad else 0)
