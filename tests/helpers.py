"""Shared test helpers: golden fixtures, error metrics, GPU upload/run glue."""
import json
import os

import numpy as np

from brimkern_amd import layout

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PLANES = {"q8": ("codes", "sc"), "q4": ("nib", "sc", "mn"), "q3": ("lo", "hi", "sc", "mn")}

# Output bar from the task: max relative error 1e-3 with f32 accumulation, measured normwise
# (max|y - r| / max|r|), plus the componentwise bound |y - r| <= tol * sum|x*w| (+ f32 floor).
REL_TOL = 1e-3


def load_golden():
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        meta = json.load(f)
    raw = np.fromfile(os.path.join(GOLDEN, "golden.bin"), dtype=np.uint8)

    def get(span, dtype):
        o, n = span
        return raw[o:o + n].view(dtype).copy()

    cases = []
    for c in meta["cases"]:
        cases.append(dict(c, x=get(c["x"], np.float32), blob=get(c["blob"], np.uint8),
                          y=get(c["y"], np.float32), deq=get(c["deq"], np.float32)))
    m = meta["moe"]
    moe = dict(m, x=get(m["x"], np.float32), blob=get(m["blob"], np.uint8), y=get(m["y"], np.float32),
               row_off=np.array(m["row_off"], np.int32))
    return cases, moe


def normwise_rel(y, r):
    y = np.asarray(y, np.float64).ravel()
    r = np.asarray(r, np.float64).ravel()
    den = np.abs(r).max() if r.size else 0.0
    if den == 0:
        return float(np.abs(y - r).max()) if r.size else 0.0
    return float(np.abs(y - r).max() / den)


def componentwise_ok(y, r, absden, tol=REL_TOL):
    y = np.asarray(y, np.float64).ravel()
    r = np.asarray(r, np.float64).ravel()
    d = np.asarray(absden, np.float64).ravel()
    return bool(np.all(np.abs(y - r) <= tol * d + 1e-30))


def moe_oracle_abs(x, row_off, t, E, K, N):
    """The expert-grouped q4 reference (per expert, the reference matmul of its rows and its [N, K]
    planes, as oracle.moe_matmul_t_q4 computes it) with the componentwise denominator sum |x w| of every
    output: (y [R, N], den [R, N])."""
    import oracle as O
    x = np.asarray(x, np.float32).reshape(-1, K)
    R = int(row_off[E])
    y = np.zeros((R, N), np.float32)
    den = np.zeros((R, N), np.float64)
    gq = N * K // 32
    for e in range(E):
        a, b = int(row_off[e]), int(row_off[e + 1])
        if b == a:
            continue
        ye, de = O.matmul_t_q4(np.ascontiguousarray(x[a:b]), t["nib"][e * N * K // 2:(e + 1) * N * K // 2],
                               t["sc"][e * gq:(e + 1) * gq], t["mn"][e * gq:(e + 1) * gq], b - a, K, N, absden=True)
        y[a:b], den[a:b] = ye, de
    return y, den


class Gpu:
    """Upload planes / run the C-ABI matmuls on one context."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.bufs = []

    def up(self, a):
        b = self.ctx.upload(np.ascontiguousarray(a))
        self.bufs.append(b)
        return b

    def planes(self, fmt, t):
        """Upload a packed blob once; return device addresses of its planes."""
        n = t["N"] * t["K"]
        blob = layout.pack(fmt, t) if "blob" not in t else t["blob"]
        buf = self.up(blob)
        return [buf.offset(layout.plane_offsets(fmt, n)[k][0]) for k in PLANES[fmt]]

    def matmul(self, fmt, x, planes, M, K, N):
        xb = self.up(np.asarray(x, np.float32)) if M * K else None
        yb = self.ctx.alloc(max(M * N, 1) * 4)
        self.bufs.append(yb)
        fn = {"q8": self.ctx.matmul_t_q8, "q4": self.ctx.matmul_t_q4, "q3": self.ctx.matmul_t_q3}[fmt]
        fn(xb, *planes, yb, M, K, N)
        return self.ctx.download(yb, np.float32, M * N).reshape(M, N)

    def dequant(self, fmt, planes, n):
        ob = self.ctx.alloc(max(n, 1) * 4)
        self.bufs.append(ob)
        fn = {"q8": self.ctx.dequant_q8, "q4": self.ctx.dequant_q4, "q3": self.ctx.dequant_q3}[fmt]
        fn(*planes, ob, n)
        return self.ctx.download(ob, np.float32, n)

    def free(self):
        for b in self.bufs:
            self.ctx.free(b)
        self.bufs.clear()
