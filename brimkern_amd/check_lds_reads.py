"""Build-time check of the GEMM kernels' inline-asm LDS reads (brik_gemm*, gemm.hip).

The multiply loop issues its LDS reads as inline asm (gemm.hip: ds_read_b128 / ds_read_u16, then
lds_wait and tie), so the compiler does not know that their destination registers are written
asynchronously. Correctness then rests on register allocation: no instruction may read or write a
destination register of such a read before the next `s_waitcnt lgkmcnt(0)`. This script disassembles the
built code object (llvm-objdump, our own build) and checks that, scanning each kernel's instructions in
address order across branches (conservative: a wait reached on any path ends the window only when it is
also the next wait in address order).

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


def check(disasm: str) -> list:
    """Violations in `disasm` (llvm-objdump -d text) of the kernels _checked selects."""
    out = []
    fn = None
    pending = {}
    for raw in disasm.split("\n"):
        m = re.match(r"^[0-9a-f]+ <([^>]+)>:", raw)
        if m:
            fn, pending = m.group(1), {}
            continue
        if fn is None or not _checked(fn):
            continue
        line = raw.split("//")[0].strip()
        if not line:
            continue
        if line.startswith("s_waitcnt") and "lgkmcnt(0)" in line:
            pending = {}
            continue
        parts = line.split(None, 1)
        ops = [o.strip().split()[0] for o in parts[1].split(",") if o.strip()] if len(parts) > 1 else []
        used = set()
        for o in ops:
            used |= _regs(o)
        hit = used & set(pending)
        if hit and not parts[0].startswith("ds_read"):
            out.append(f"{fn}: '{line}' touches v{sorted(hit)} before the LDS read that writes it has been waited for")
        if parts[0] in ASM_READS and ops:
            for r in _regs(ops[0]):
                pending[r] = line
    return out


def check_file(path: str) -> list:
    if not os.path.exists(OBJDUMP):
        return []
    text = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", path], capture_output=True, text=True,
                          check=True).stdout
    return check(text)


if __name__ == "__main__":
    bad = check_file(sys.argv[1])
    for b in bad[:20]:
        print(b)
    print(f"{len(bad)} violation(s)")
    sys.exit(1 if bad else 0)
