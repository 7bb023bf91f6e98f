"""GPU parity of the linked GLU plans (brik_gemv_plan_create_glu): the gate/up launch computes rows of
the same indices of both matrices in one block and writes the staged image of act(gate) * up for down,
which copies it instead of transforming its input in every block.

Against the two ordinary plans {gate, up} and {down with gate = gate.y, x = up.y} (the feed-forward
half of recordLayerKV, kernels.ts:1726-1741), whose own parity against the oracle is tested in
test_gpu_fused.py: down.y must be bit-identical to the ordinary down plan's on the same gate.y and
up.y (the image equals the consumer's own staging), and gate.y / up.y equal the ordinary plan's within
f32 rounding (the pair block has 8 waves, so the RMSNorm factor is summed in another order). Past 256
groups of down's input the pair launch writes the image of whole groups for the first multiple of 256
and the consumer stages the rest from the values the launch's 8-row blocks write (shapes below). One case
also checks the chain against the oracle directly. Non-finite gate / up outputs must send down through
the exact path, as the self-staged input does.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_OPT_GEMV_VARIANT
from helpers import Gpu, PLANES, normwise_rel

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def job(gpu, fmt, planes, xb, yb, K, N, **fuse):
    names = {"q8": ("p0", "sc"), "q4": ("p0", "sc", "mn"), "q3": ("p0", "p1", "sc", "mn")}[fmt]
    j = dict(zip(names, planes), x=xb, y=yb, K=K, N=N)
    j.update(fuse)
    return j


class Ffn:
    """gate / up [F, D] on one input row (optionally RMSNorm-fused), down [D, F] on act(gate) * up."""

    def __init__(self, gpu, fmt, D, F, seed, norm=True, gelu=False, res=True, tensors=None):
        self.gpu, self.fmt, self.D, self.F = gpu, fmt, D, F
        self.t = tensors or {n: synth.tensor(fmt, seed + i, N, K)
                             for i, (n, K, N) in enumerate([("gate", D, F), ("up", D, F), ("down", F, D)])}
        self.planes = {n: gpu.planes(fmt, t) for n, t in self.t.items()}
        self.x = synth.normal(seed + 10, D) * 2
        self.w = synth.normal(seed + 11, D) * 0.2 + 1
        self.res = synth.normal(seed + 12, D)
        self.xb, self.wb, self.rb = gpu.up(self.x), gpu.up(self.w), gpu.up(self.res)
        self.norm, self.gelu, self.with_res = norm, gelu, res

    def jobs(self):
        g = self.gpu
        out = {n: g.up(np.full(N, np.nan, np.float32)) for n, N in (("gate", self.F), ("up", self.F), ("y", self.D))}
        fuse = dict(norm_w=self.wb, eps=1e-6) if self.norm else {}
        jg = job(g, self.fmt, self.planes["gate"], self.xb, out["gate"], self.D, self.F, **fuse)
        ju = job(g, self.fmt, self.planes["up"], self.xb, out["up"], self.D, self.F, **fuse)
        dfuse = dict(gate=out["gate"], gelu=self.gelu)
        if self.with_res:
            dfuse["res"] = self.rb
        jd = job(g, self.fmt, self.planes["down"], out["up"], out["y"], self.F, self.D, **dfuse)
        return jg, ju, jd, out

    def read(self, out):
        c = self.gpu.ctx
        return {n: c.download(b, np.float32, b.nbytes // 4) for n, b in out.items()}

    def run_linked(self, runs=1):
        """The linked pair; "y_plain": the ordinary down plan on the pair's gate.y and up.y, on the GEMV
        variant the pair's consumer runs (variant 6: 4-row blocks, 64 lanes per row), so that the two differ only in where the staged image comes from. q8 has no pair kernel:
        its "pair" is two ordinary plans, compared with an ordinary plan as it is."""
        jg, ju, jd, out = self.jobs()
        gu, dn = self.gpu.ctx.gemv_plan_glu(self.fmt, jg, ju, jd)
        for _ in range(runs):
            gu.run()
            dn.run()
        out["y_plain"] = self.gpu.up(np.full(self.D, np.nan, np.float32))
        self.gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, 0 if self.fmt == "q8" else 1 + 6)
        try:
            plain = self.gpu.ctx.gemv_plan(self.fmt, [dict(jd, y=out["y_plain"])])
        finally:
            self.gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, 0)
        plain.run()
        r = self.read(out)
        plain.destroy()
        gu.destroy()
        dn.destroy()
        return r

    def run_plain(self):
        jg, ju, jd, out = self.jobs()
        p1 = self.gpu.ctx.gemv_plan(self.fmt, [jg, ju])
        p2 = self.gpu.ctx.gemv_plan(self.fmt, [jd])
        p1.run()
        p2.run()
        r = self.read(out)
        p1.destroy()
        p2.destroy()
        return r


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def check_pair(a, b):
    """a: linked outputs, b: ordinary plans' outputs."""
    assert same_bits(a["y"], a["y_plain"])
    for n in ("gate", "up"):
        fa, fb = np.isfinite(a[n]), np.isfinite(b[n])
        assert np.array_equal(fa, fb) and np.array_equal(np.isnan(a[n]), np.isnan(b[n])), n
        assert np.array_equal(a[n][~fa & ~np.isnan(a[n])], b[n][~fb & ~np.isnan(b[n])]), n
        assert normwise_rel(a[n][fa], b[n][fb]) <= 1e-6, n
    fa = np.isfinite(a["y"])
    assert np.array_equal(fa, np.isfinite(b["y"]))
    if fa.any():
        assert normwise_rel(a["y"][fa], b["y"][fa]) <= 1e-5


@pytest.mark.parametrize("fmt", ["q4", "q3", "q8"])
# (2560, 9728): 304 groups of down's input on 256 CUs, so the pair launch writes the image of the first
# 256 and runs the last 48 in 8-row blocks that the consumer stages itself; (256, 8448) and
# (128, 8224): 264 and 257 groups, a remainder of 8 and of 1
@pytest.mark.parametrize("shape", [(2560, 9728), (256, 96), (64, 32), (512, 1024), (256, 8448), (128, 8224)])
def test_glu_matches_ordinary_plans(gpu, fmt, shape):
    D, F = shape
    f = Ffn(gpu, fmt, D, F, 300)
    a, b = f.run_linked(runs=2), f.run_plain()
    check_pair(a, b)


@pytest.mark.parametrize("fmt", ["q4", "q3"])
@pytest.mark.parametrize("variant", ["geglu", "no_norm_no_res"])
@pytest.mark.parametrize("F", [2048, 8448])     # 8448: 264 groups, the last 8 staged by the consumer
def test_glu_variants_match(gpu, fmt, variant, F):
    f = Ffn(gpu, fmt, 1024 if F == 2048 else 256, F, 310, norm=variant != "no_norm_no_res",
            gelu=variant == "geglu", res=variant != "no_norm_no_res")
    a, b = f.run_linked(), f.run_plain()
    check_pair(a, b)


@pytest.mark.parametrize("fmt", ["q4", "q3"])
def test_glu_against_oracle(gpu, fmt):
    D, F = 1024, 1536
    f = Ffn(gpu, fmt, D, F, 320)
    got = f.run_linked()
    n2 = O.rmsnorm(f.x, f.w, 1, D, 1e-6)
    def mm(x, t, K, N):
        return getattr(O, f"matmul_t_{fmt}")(np.asarray(x, np.float32), *[t[p] for p in PLANES[fmt]], 1, K, N).ravel()
    assert normwise_rel(got["gate"], mm(n2, f.t["gate"], D, F)) <= TOL
    assert normwise_rel(got["up"], mm(n2, f.t["up"], D, F)) <= TOL
    g = O.swiglu(got["gate"], got["up"])
    assert normwise_rel(got["y"], f.res + mm(g, f.t["down"], F, D)) <= TOL


@pytest.mark.parametrize("fmt", ["q4", "q3"])
@pytest.mark.parametrize("where", ["gate_row", "input", "tail_gate_row", "tail_input"])
def test_glu_non_finite(gpu, fmt, where):
    """An infinite scale in one gate row (one group of down's input non-finite) or an Inf in the shared
    input (every gate / up output non-finite) must put down on the exact path, as with a self-staged
    input: the same outputs, NaN and Inf included, as the unlinked plans. tail_gate_row: the row lies
    in the groups the consumer stages itself (F = 9728: groups 256-303); tail_input: the Inf input at
    that size (the exact path of the pair launch's 8-row blocks too)."""
    D, F = 512, 9728 if where.startswith("tail") else 1024
    t = {n: synth.tensor(fmt, 330 + i, N, K) for i, (n, K, N) in enumerate([("gate", D, F), ("up", D, F),
                                                                            ("down", F, D)])}
    if where in ("gate_row", "tail_gate_row"):
        row = 9000 if where == "tail_gate_row" else 77
        sc = t["gate"]["sc"].copy()
        sc[(row * D) // 32 + 3] = 0x7C00         # +Inf scale in one row of gate
        t["gate"]["sc"] = sc
    f = Ffn(gpu, fmt, D, F, 330, tensors=t)
    if where in ("input", "tail_input"):
        f.x[5] = np.inf
        f.xb = gpu.up(f.x)
    a, b = f.run_linked(), f.run_plain()
    check_pair(a, b)
    assert not np.isfinite(a["gate"]).all()


def test_glu_destroy_order_and_rerun(gpu):
    """The plans share the image: the producer may be destroyed first, and the consumer still reads
    the image of the producer's last run."""
    f = Ffn(gpu, "q4", 512, 1024, 340)
    jg, ju, jd, out = f.jobs()
    gu, dn = gpu.ctx.gemv_plan_glu("q4", jg, ju, jd)
    gu.run()
    dn.run()
    y1 = gpu.ctx.download(out["y"], np.float32, f.D)
    gu.destroy()
    gpu.ctx.h2d(out["y"], np.zeros(f.D, np.float32))
    dn.run()                                     # res is not y: the same result again
    y2 = gpu.ctx.download(out["y"], np.float32, f.D)
    dn.destroy()
    assert same_bits(y1, y2)


def test_glu_rejects_mismatched_jobs(gpu):
    f = Ffn(gpu, "q4", 256, 512, 350)
    jg, ju, jd, out = f.jobs()
    bad = [
        (dict(jg, K=128), ju, jd),                          # gate and up differ in K
        (jg, dict(ju, x=f.rb), jd),                         # different inputs
        (jg, dict(ju, norm_w=None), jd),                    # different fusion
        (jg, dict(ju, y=jg["y"]), jd),                      # one output for both
        (jg, ju, dict(jd, x=jg["y"])),                      # down does not read up
        (jg, ju, dict(jd, gate=None)),                      # down has no gate
        (jg, ju, dict(jd, norm_w=f.wb)),                    # down with RMSNorm
        (jg, ju, dict(jd, K=256)),                          # down.K != N
    ]
    for g, u, d in bad:
        with pytest.raises(BrikError) as e:
            gpu.ctx.gemv_plan_glu("q4", g, u, d)
        assert e.value.code == BRIK_EINVAL
