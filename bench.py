#!/usr/bin/env python3
"""bench.py — q4 decode GEMV HBM GB/s at Qwen3-4B shapes on one MI355X (+ the other benchmarked configurations).

Headline (``value``): the full Qwen3-4B q4 GEMV layer set at M=1 (K=2560 -> N in {4096, 1024, 1024,
9728, 9728}; K=9728 -> N=2560) for all 36 layers — 216 matrices, 2.04 GB of distinct packed weights,
8x the 256 MB Infinity Cache, so every step streams from HBM — executed as one grouped GEMV plan
(its staging launch and one GEMV launch per step). A step = one pass over the 216 matrices.
``value`` = algorithmic bytes (packed W + x + y) per step / step time.

Also measured and reported under ``extra`` (same run, same process): the per-matrix single-launch
GEMV at each Qwen3-4B shape, the q8 GEMV (cfg 1), the q3 LM head (cfg 3), the prefill q4 GEMM
TFLOP/s (cfg 4) and the MoE expert-grouped q4 GEMM (cfg 5); every one rotates enough distinct weight
copies to exceed the Infinity Cache.

``cpu_baseline``: the reference's CPU matmul restated in JavaScript (oracle/cpuref.js: dequantize the
tensor, f64-accumulated dot per output), run by node on this host on one Qwen3-4B layer set (M=1,
the same six shapes), single-threaded, repeated to a sample of about 15 s; value = mean rate.

``roofline``: ``achieved`` = algorithmic bytes per step / the step's average duration (HIP events on
the library's stream). A step is the plan's staging launch (each distinct input row staged once) and
its GEMV launch, both inside the timed region. ``traffic`` = HBM bytes per step from two rocprofv3
counter passes (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch) run as child processes before this
process opens the GPU, each scaled by the same counter's reading for a device copy of known size.

Timing: HIP events on the library's stream bracket exactly ``--steps`` steps after ``--warmup``
untimed ones, with a device synchronization on both sides. Before the headline's warmup steps the
same step runs untimed for ``--settle`` seconds: a freshly started process meets the GPU's clocks in
a transient (on the box, the first ~10 ms of back-to-back launches vary by +-15 % before holding
steady), and the headline is the steady-state rate a decode loop sees.
"""
import argparse
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
from brimkern_amd.capi import BRIK_OPT_PATH, BRIK_OPT_SPLITK, PATH_AUTO, PATH_GEMV, PATH_GEMM  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16
QWEN3_4B = [("q", 2560, 4096), ("k", 2560, 1024), ("v", 2560, 1024),
            ("gate", 2560, 9728), ("up", 2560, 9728), ("down", 9728, 2560)]
LAYERS = 36


def q_bytes(fmt, N, K):
    from brimkern_amd import layout
    return layout.byte_length(fmt, N * K)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


MIN_TIMED_MS = 20.0           # timed work of an `extra` line, at least (time_loop_min)
ROTATE_BYTES = 512 << 20        # distinct weight copies a per-call timing cycles through: 2x the MALL
SMALL_M = (2, 4, 8, 15)


def synth_rows(K, M):
    from brimkern_amd import synth
    return synth.normal(900 + K, M * K)


class Replicas:
    """``count`` device copies (distinct addresses) of one packed tensor; returns plane addresses."""

    def __init__(self, ctx, fmt, t, count):
        from brimkern_amd import layout
        self.fmt, self.N, self.K, self.tensor = fmt, t["N"], t["K"], t
        blob = layout.pack(fmt, t)
        self.stride = (blob.size + 255) // 256 * 256
        self.buf = ctx.alloc(self.stride * count)
        ctx.h2d(self.buf, blob)
        for i in range(1, count):
            ctx._check(ctx.lib.brik_d2d(ctx.handle, ctx_p(self.buf.ptr + i * self.stride), ctx_p(self.buf.ptr),
                                        blob.size))
        self.offs = layout.plane_offsets(fmt, self.N * self.K)
        self.count = count

    def planes(self, i):
        base = self.buf.ptr + i * self.stride
        names = {"q8": ("codes", "sc"), "q4": ("nib", "sc", "mn"), "q3": ("lo", "hi", "sc", "mn")}[self.fmt]
        return [base + self.offs[k][0] for k in names]


def ctx_p(v):
    import ctypes
    return ctypes.c_void_p(v)


def time_loop(ctx, fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    ctx.sync()
    ctx.timer_begin()
    for i in range(steps):
        fn(i)
    ms = ctx.timer_end()
    ctx.sync()
    return ms / steps


def time_loop_min(ctx, fn, steps, warmup, min_ms=MIN_TIMED_MS):
    """time_loop for the `extra` lines: if `steps` calls take less than min_ms, time again with enough
    calls to fill it. The queue starts empty after the warmup's synchronize, and over a few milliseconds
    that start-up latency (about 0.1 ms here) still shows in the mean."""
    ms = time_loop(ctx, fn, steps, warmup)
    if ms * steps < min_ms:
        ms = time_loop(ctx, fn, int(math.ceil(min_ms / max(ms, 1e-4))), 0)
    return ms


GRAPHS = True     # False under --no-graph: the graph-replayed lines are timed eagerly instead


def time_graph(ctx, fn, count, min_calls=256, min_ms=MIN_TIMED_MS):
    """fn(i), i = 0 .. n-1 (n >= count, so every weight copy appears), recorded into one graph and
    replayed until at least min_ms of GPU time; returns ms per call. This is the GPU-side rate of
    back-to-back launches, as a decode step recorded once and replayed issues them (the reference
    records a layer's matmuls into one command encoder); a Python loop of calls is bound by the host
    for launches this short. With GRAPHS off (--no-graph, for profiler runs) the calls run eagerly."""
    n = max(count, min_calls)
    if not GRAPHS:
        return time_loop_min(ctx, fn, n, count)
    fn(0)
    ctx.sync()              # workspaces at their size before the capture (which refuses growth)
    ctx.graph_begin()
    for i in range(n):
        fn(i)
    g = ctx.graph_end()
    try:
        g.launch()
        ctx.sync()
        ctx.timer_begin()
        g.launch()
        one = ctx.timer_end()
        reps = max(2, int(math.ceil(min_ms / max(one, 1e-3))))
        ctx.sync()
        ctx.timer_begin()
        for _ in range(reps):
            g.launch()
        ms = ctx.timer_end()
        ctx.sync()
    finally:
        g.destroy()
    return ms / (reps * n)


def settle(ctx, fn, seconds):
    """Run ``fn`` untimed until ``seconds`` of wall time have passed (GPU clocks reach steady state)."""
    if seconds <= 0:
        return
    t0 = time.time()
    i = 0
    while time.time() - t0 < seconds:
        for _ in range(16):
            fn(i)
            i += 1
        ctx.sync()


HEAD_X_SEED = {2560: 101, 9728: 102}     # the headline's activation rows by K (shared with cpu_baseline)


def head_x(K):
    from brimkern_amd import synth
    return synth.normal(HEAD_X_SEED[K], K)


def build_layer_plan(ctx, layers):
    """One grouped GEMV plan over ``layers`` distinct copies of the Qwen3-4B q4 layer set."""
    from brimkern_amd import synth
    reps, jobs, nbytes = {}, [], 0
    xa = ctx.upload(head_x(2560))
    xd = ctx.upload(head_x(9728))
    ybuf = ctx.alloc(4 * layers * sum(n for _, _, n in QWEN3_4B))
    yo = 0
    for si, (name, K, N) in enumerate(QWEN3_4B):
        reps[name] = Replicas(ctx, "q4", synth.q4_tensor(200 + si, N, K), layers)
    for l in range(layers):
        for name, K, N in QWEN3_4B:
            nib, sc, mn = reps[name].planes(l)
            jobs.append({"x": xd if K == 9728 else xa, "p0": nib, "sc": sc, "mn": mn,
                         "y": ybuf.ptr + 4 * yo, "K": K, "N": N})
            yo += N
            nbytes += q_bytes("q4", N, K) + 4 * K + 4 * N
    plan = ctx.gemv_plan("q4", jobs)
    return plan, {"reps": reps, "xa": xa, "xd": xd, "ybuf": ybuf, "nbytes": nbytes}


def gemv_layer_set(ctx, steps, warmup, layers, settle_s, graph_replay=True):
    plan, b = build_layer_plan(ctx, layers)
    reps, xa, xd, ybuf, nbytes = b["reps"], b["xa"], b["xd"], b["ybuf"], b["nbytes"]
    settle(ctx, lambda i: plan.run(), settle_s)
    ms = time_loop(ctx, lambda i: plan.run(), steps, warmup)
    # the last timed step's outputs: all 216 matrices, checked against the CPU reference later
    y_head = ctx.download(ybuf, np.float32, ybuf.nbytes // 4)
    plan.destroy()
    # per-shape single launches and small-M calls, each rotating over distinct weight copies totalling
    # at least twice the 256 MB last-level cache (so every call streams its weights from HBM)
    single, small_m = {}, {}
    for name, K, N in QWEN3_4B:
        tb = q_bytes("q4", N, K)
        count = max(layers, -(-ROTATE_BYTES // tb))
        extra = Replicas(ctx, "q4", reps[name].tensor, count) if count > layers else reps[name]
        x = xd if K == 9728 else xa
        xm = ctx.upload(synth_rows(K, max(SMALL_M)))
        yb = ctx.alloc(4 * N * max(SMALL_M))

        def one(i, M=1, r=extra, yb=yb, K=K, N=N, count=count):
            nib, sc, mn = r.planes(i % count)
            ctx.matmul_t_q4(x if M == 1 else xm, nib, sc, mn, yb, M, K, N)
        lms = time_graph(ctx, one, count)
        ems = time_loop_min(ctx, one, max(4 * layers, count), count)
        bb = tb + 4 * K + 4 * N
        single[f"{name}_K{K}_N{N}"] = {"us": round(lms * 1e3, 2), "GBps": round(bb / (lms * 1e-3) / 1e9, 1),
                                       "eager_us": round(ems * 1e3, 2), "copies": count}
        small_m_rows(ctx, small_m, f"{name}_K{K}_N{N}", tb, count, one)
        if extra is not reps[name]:
            ctx.free(extra.buf)
        ctx.free(xm)
        ctx.free(yb)
    fused = decode_layers_fused(ctx, reps, layers, steps, warmup, graph_replay)
    for r in reps.values():
        ctx.free(r.buf)
    ctx.free(ybuf)
    return ms, nbytes, single, fused, small_m, y_head


def small_m_rows(ctx, small_m, key, tb, count, one):
    """``one(i, M)`` at M in SMALL_M on each path (auto, GEMV, tiled, split-K), graph-replayed."""
    for M in SMALL_M:
        row = {}
        for label, path, sk in (("auto", PATH_AUTO, 0), ("gemv", PATH_GEMV, 0), ("tiled", PATH_GEMM, 1),
                                ("splitk", PATH_GEMM, 2)):
            ctx.set_option(BRIK_OPT_PATH, path)
            ctx.set_option(BRIK_OPT_SPLITK, sk)
            try:
                ms_m = time_graph(ctx, lambda i, M=M: one(i, M), count, min_calls=64)
            finally:
                ctx.set_option(BRIK_OPT_PATH, PATH_AUTO)
                ctx.set_option(BRIK_OPT_SPLITK, 0)
            row[label + "_us"] = round(ms_m * 1e3, 2)
        row["weight_GBps"] = round(tb / (row["auto_us"] * 1e-6) / 1e9, 1)
        small_m.setdefault(f"M{M}", {})[key] = row


def small_m_formats(ctx):
    """The few-row lines for q8 and q3 weights at three Qwen3-4B shapes (k/v, gate, down), graph-replayed."""
    from brimkern_amd import synth
    out = {}
    for fmt in ("q8", "q3"):
        rows = {}
        for name, K, N in (("k", 2560, 1024), ("gate", 2560, 9728), ("down", 9728, 2560)):
            t = synth.tensor(fmt, 250, N, K)
            tb = q_bytes(fmt, N, K)
            count = max(2, -(-ROTATE_BYTES // tb))
            r = Replicas(ctx, fmt, t, count)
            xm = ctx.upload(synth_rows(K, max(SMALL_M)))
            yb = ctx.alloc(4 * N * max(SMALL_M))
            fn = {"q8": ctx.matmul_t_q8, "q3": ctx.matmul_t_q3}[fmt]

            def one(i, M, r=r, xm=xm, yb=yb, K=K, N=N, count=count, fn=fn):
                fn(xm, *r.planes(i % count), yb, M, K, N)
            small_m_rows(ctx, rows, f"{name}_K{K}_N{N}", tb, count, one)
            for bb in (r.buf, xm, yb):
                ctx.free(bb)
        out[fmt] = rows
    return out


def decode_layers_fused(ctx, reps, layers, steps, warmup, graph_replay=True):
    """The matmul side of ``layers`` Qwen3-4B decoder layers as recordLayerKV chains it
    (kernels.ts:1701-1741), four fused plans per layer: q/k/v on rmsnorm(x), wo + residual, gate/up on
    rmsnorm(h), down on swiglu(gate, up) + residual; layer l + 1 reads layer l's output. Attention is
    outside this library: its output is a fixed seeded vector."""
    from brimkern_amd import synth
    d, qd, kvd, ffn = 2560, 4096, 1024, 9728
    attn = ctx.upload(synth.normal(110, qd))
    an, fn = ctx.upload(synth.normal(111, d) * 0.1 + 1), ctx.upload(synth.normal(112, d) * 0.1 + 1)
    xs = [ctx.upload(synth.normal(113, d))] + [ctx.alloc(4 * d) for _ in range(layers)]
    tmp = {n: ctx.alloc(4 * N) for n, N in (("q", qd), ("k", kvd), ("v", kvd), ("h", d), ("gate", ffn), ("up", ffn))}
    shapes = {n: (K, N) for n, K, N in QWEN3_4B + [("o", qd, d)]}
    reps = dict(reps, o=Replicas(ctx, "q4", synth.q4_tensor(114, d, qd), layers))   # wo, not in the GEMV layer set

    def j(name, l, x, y, **f):
        nib, sc, mn = reps[name].planes(l)
        K, N = shapes[name]
        return dict(x=x, p0=nib, sc=sc, mn=mn, y=y, K=K, N=N, **f)
    plans, nbytes = [], 0
    for l in range(layers):
        x, y = xs[l], xs[l + 1]
        # gate/up and down as the linked GLU pair: the gate/up launch writes down's staged input
        glu = ctx.gemv_plan_glu("q4", j("gate", l, tmp["h"], tmp["gate"], norm_w=fn, eps=1e-6),
                                j("up", l, tmp["h"], tmp["up"], norm_w=fn, eps=1e-6),
                                j("down", l, tmp["up"], y, gate=tmp["gate"], res=tmp["h"]))
        plans += [ctx.gemv_plan("q4", [j(n, l, x, tmp[n], norm_w=an, eps=1e-6) for n in ("q", "k", "v")]),
                  ctx.gemv_plan("q4", [j("o", l, attn, tmp["h"], res=x)]), *glu]
        nbytes += sum(q_bytes("q4", N, K) for K, N in shapes.values())

    def step(i):
        for p in plans:
            p.run()
    ms_eager = time_loop(ctx, step, max(2, steps // 4), max(1, warmup // 2))
    ms = None
    if graph_replay:
        # the same launches recorded once and replayed (brik_graph_*), as the reference records a
        # layer into one command encoder
        ctx.graph_begin()
        step(0)
        graph = ctx.graph_end()
        ms = time_loop(ctx, lambda i: graph.launch(), steps, warmup)
        graph.destroy()
    for p in plans:
        p.destroy()
    for b in [attn, an, fn, reps["o"].buf] + xs + list(tmp.values()):
        ctx.free(b)
    replay = "one recorded graph per step"
    if ms is None:
        ms, replay = ms_eager, "eager (graph replay skipped: --no-graph)"
    return {"us_per_layer": round(ms * 1e3 / layers, 2), "weight_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "replay": replay,
            "eager_us_per_layer": round(ms_eager * 1e3 / layers, 2), "launches_per_layer": 4, "layers": layers,
            "fused": "rmsnorm -> q/k/v, wo + residual, rmsnorm -> gate/up (+ staged swiglu image of the "
                     "first 256 groups, swiglu values of the rest), down (copies the image, stages the rest) "
                     "+ residual"}


def gemv_single_cfg(ctx, fmt, K, N, seed, steps, warmup, cache_bytes=768 << 20):
    from brimkern_amd import synth
    t = synth.tensor(fmt, seed, N, K)
    tb = q_bytes(fmt, N, K)
    copies = max(2, -(-cache_bytes // tb))
    r = Replicas(ctx, fmt, t, copies)
    x = ctx.upload(synth.normal(seed + 1, K))
    y = ctx.alloc(4 * N)
    fn = {"q8": ctx.matmul_t_q8, "q4": ctx.matmul_t_q4, "q3": ctx.matmul_t_q3}[fmt]
    call = lambda i: fn(x, *r.planes(i % copies), y, 1, K, N)   # noqa: E731
    ms = time_graph(ctx, call, copies)
    ems = time_loop_min(ctx, call, max(steps, copies), copies)
    b = tb + 4 * K + 4 * N
    for bb in (r.buf, x, y):
        ctx.free(bb)
    return {"us": round(ms * 1e3, 2), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
            "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "eager_us": round(ems * 1e3, 2),
            "copies": copies, "timing": "graph-replayed back-to-back calls (eager_us: a Python loop of calls)"}


def lm_head_topk_cfg3(ctx, steps, warmup, gemv_us, cache_bytes=768 << 20):
    """The cfg 3 q3 LM head fused with the sampling pre-work (softcap 30, penalty 1.15 over 40 recent
    ids, top 64), as decodeTopKQ8 records them; and the passes alone over 151936 logits."""
    from brimkern_amd import synth
    K, N, k = 2560, 151936, 64
    t = synth.tensor("q3", 700, N, K)
    copies = max(2, -(-cache_bytes // q_bytes("q3", N, K)))
    r = Replicas(ctx, "q3", t, copies)
    x = ctx.upload(synth.normal(701, K))
    rec = ctx.upload(np.unique((synth.uniform(702, 40) * N).astype(np.int32)))
    nrec = int(rec.nbytes // 4)
    out = ctx.alloc(8 * k)
    ms = time_loop_min(ctx, lambda i: ctx.lm_head_topk("q3", x, r.planes(i % copies), K, N, rec, nrec, 1.15, 30.0, k,
                                                  out, out.offset(4 * k)), max(steps, copies), copies)
    logits = ctx.upload(synth.normal(703, N) * 4)
    ms_p = time_loop_min(ctx, lambda i: ctx.logits_topk(logits, N, rec, nrec, 1.15, 30.0, k, out, out.offset(4 * k)),
                     steps, warmup)
    for bb in (r.buf, x, rec, out, logits):
        ctx.free(bb)
    return {"us": round(ms * 1e3, 2), "passes_alone_us": round(ms_p * 1e3, 2),
            "over_gemv_us": round(ms * 1e3 - gemv_us, 2), "readback_bytes": 8 * k,
            "launches": "brik_gemv_stage1_q3 + brik_gemvh_q3 (head GEMV, softcap / penalty / 16-logit maxima "
                        "in its epilogue) + brik_topk_select; passes_alone: brik_topk_prep + brik_topk_select"}


def quantize_f1(ctx, steps, warmup):
    """The GPU encoders (quantizeQ* byte-exact) on a Qwen3-4B gate matrix, 9728 x 2560 f32 -> packed
    planes: algorithmic bytes = 4 n read + the packed planes written. Two source copies alternate
    (each 100 MB, so together beyond the 256 MB last-level cache)."""
    from brimkern_amd import layout, synth
    n = 9728 * 2560
    src = [ctx.upload(synth.normal(900 + i, n)) for i in range(3)]
    out = {}
    planes_of = {"q8": ("codes", "sc"), "q4": ("nib", "sc", "mn"), "q3": ("lo", "hi", "sc", "mn")}
    for fmt in ("q8", "q4", "q3"):
        ob = ctx.alloc(layout.byte_length(fmt, n))
        offs = layout.plane_offsets(fmt, n)
        pl = [ob.offset(offs[p][0]) for p in planes_of[fmt]]
        ms = time_loop_min(ctx, lambda i: ctx.quantize(fmt, src[i % 3], pl, n), steps, warmup)
        b = 4 * n + layout.byte_length(fmt, n)
        out[fmt] = {"us": round(ms * 1e3, 2), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
                    "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "Gelem_per_s": round(n / (ms * 1e-3) / 1e9, 1)}
        ctx.free(ob)
    for bb in src:
        ctx.free(bb)
    out["elements"] = n
    out["kernels"] = "brik_encode_q8 / brik_encode_q4 / brik_encode_q3"
    return out


def conv_f4(ctx, steps, warmup):
    """A UNet-sized 3x3 convolution with a q4 weight (Cin = Cout = 320 on a 64 x 64 latent, stride 1,
    pad 1): the implicit MFMA GEMM path and, for comparison, the direct kernel (the reference's
    conv2d_direct_q4 scheme: one output per thread)."""
    from brimkern_amd import layout, synth
    from brimkern_amd.capi import BRIK_OPT_PATH
    Cin, H, W, Cout, k = 320, 64, 64, 320, 3
    nw = Cout * Cin * k * k
    t = synth.q4_tensor(950, Cout, Cin * k * k)
    wb = ctx.upload(layout.pack("q4", t))
    offs = layout.plane_offsets("q4", nw)
    planes = [wb.offset(offs[p][0]) for p in ("nib", "sc", "mn")]
    x = ctx.upload(synth.normal(951, Cin * H * W))
    b = ctx.upload(synth.normal(952, Cout))
    y = ctx.alloc(4 * Cout * H * W)
    flops = 2.0 * Cout * H * W * Cin * k * k
    out = {}
    for name, path, st in (("implicit_gemm", 0, steps), ("direct", 1, max(2, steps // 10))):
        ctx.set_option(BRIK_OPT_PATH, path)
        ms = time_loop_min(ctx, lambda i: ctx.conv2d("q4", x, planes, b, y, Cin, H, W, Cout, k, k, 1, 1), st, 2)
        out[name] = {"us": round(ms * 1e3, 2), "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1)}
    ctx.set_option(BRIK_OPT_PATH, 0)
    for bb in (wb, x, b, y):
        ctx.free(bb)
    out["shape"] = "Cin 320, 64x64, Cout 320, 3x3, stride 1, pad 1, q4 weight"
    out["frac_of_mfma_peak"] = round(out["implicit_gemm"]["TFLOPs"] / MFMA_F16_PEAK_TFLOPS, 4)
    out["launches"] = "brik_conv_chanmax + brik_xprep_im2col3_f16 + brik_gemm_q4 (stores [Cout, pixels] + bias)"
    return out


def f16w_f4(ctx, steps, warmup, cache_bytes=768 << 20):
    """The f16-weight matmul (MATMUL_T_F16W) on the Qwen3-4B gate shape (N 9728, K 2560, W 49.8 MB):
    decode GEMV (M = 1, rotating weight copies beyond the last-level cache; HBM bytes = 2 N K + x + y)
    and prefill (M = 512, MFMA)."""
    from brimkern_amd import synth
    M, K, N = 512, 2560, 9728
    wbytes = 2 * N * K
    copies = max(2, -(-cache_bytes // wbytes))
    w = (synth.normal(960, N * K) * 0.05).astype(np.float16).view(np.uint16)
    ws = [ctx.upload(w) for _ in range(copies)]
    x = ctx.upload(synth.normal(961, M * K))
    y = ctx.alloc(4 * M * N)
    ms1 = time_loop_min(ctx, lambda i: ctx.matmul_t_f16w(x, ws[i % copies], y, 1, K, N), max(steps, copies), copies)
    b1 = wbytes + 4 * K + 4 * N
    msm = time_loop_min(ctx, lambda i: ctx.matmul_t_f16w(x, ws[i % copies], y, M, K, N), steps, warmup)
    tf = 2.0 * M * N * K / (msm * 1e-3) / 1e12
    for bb in ws + [x, y]:
        ctx.free(bb)
    return {"gemv_M1": {"us": round(ms1 * 1e3, 2), "GBps": round(b1 / (ms1 * 1e-3) / 1e9, 1),
                        "frac": round(b1 / (ms1 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "copies": copies},
            "gemm_M512": {"us": round(msm * 1e3, 2), "TFLOPs": round(tf, 1),
                          "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)},
            "kernels": "brik_gemv_f16w_v8 (M = 1); brik_xprep_f16 + brik_gemm_f16_96x1w8 (M = 512)"}


def gemm_cfg4(ctx, steps, warmup):
    from brimkern_amd import synth
    M, K, N = 512, 2560, 9728
    copies = 36
    r = Replicas(ctx, "q4", synth.q4_tensor(300, N, K), copies)
    x = ctx.upload(synth.normal(301, M * K))
    y = ctx.alloc(4 * M * N)
    ms = time_loop_min(ctx, lambda i: ctx.matmul_t_q4(x, *r.planes(i % copies), y, M, K, N), max(steps, copies), 4)
    flops = 2.0 * M * N * K
    for bb in (r.buf, x, y):
        ctx.free(bb)
    tf = flops / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1), "bound": "mfma", "peak_TFLOPs": MFMA_F16_PEAK_TFLOPS,
            "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "launches": "brik_xprep_f16 + brik_gemm_q4 per call"}


def moe_cfg5(ctx, steps, warmup):
    from brimkern_amd import synth
    T, H, E, F, TOPK = 256, 2048, 64, 768, 8
    rows, row_off = synth.moe_routing(77, T, E, TOPK)
    R = rows.size
    copies = 3
    reps = {w: Replicas(ctx, "q4", synth.q4_tensor(400 + i, E * (F if w != "down" else H), F if w == "down" else H),
                        copies) for i, w in enumerate(("gate", "up", "down"))}
    xg = ctx.upload(np.ascontiguousarray(synth.normal(401, T * H).reshape(T, H)[rows]))
    xd = ctx.upload(synth.normal(402, R * F))
    ro = ctx.upload(row_off)
    yg = ctx.alloc(4 * R * F)
    yu = ctx.alloc(4 * R * F)
    yd = ctx.alloc(4 * R * H)

    def step3(i):
        c = i % copies
        ctx.moe_matmul_t_q4(xg, ro, *reps["gate"].planes(c), yg, E, R, H, F)
        ctx.moe_matmul_t_q4(xg, ro, *reps["up"].planes(c), yu, E, R, H, F)
        ctx.moe_matmul_t_q4(xd, ro, *reps["down"].planes(c), yd, E, R, F, H)

    def step(i):     # gate and up in one launch on one staging of x (brik_moe_matmul_t_q4_x2), then down
        c = i % copies
        ctx.moe_matmul_t_q4_x2(xg, ro, reps["gate"].planes(c), yg, reps["up"].planes(c), yu, E, R, H, F)
        ctx.moe_matmul_t_q4(xd, ro, *reps["down"].planes(c), yd, E, R, F, H)
    ms3 = time_loop_min(ctx, step3, max(steps, 6), 3)
    ms = time_loop_min(ctx, step, max(steps, 6), 3)
    wbytes = 2 * q_bytes("q4", E * F, H) + q_bytes("q4", E * H, F)
    flops = 2.0 * R * (2 * H * F + F * H)
    for bb in list(r.buf for r in reps.values()) + [xg, xd, ro, yg, yu, yd]:
        ctx.free(bb)
    return {"us": round(ms * 1e3, 2), "weight_GBps": round(wbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 2), "rows": int(R),
            "max_rows_per_expert": int(np.diff(row_off).max()), "min_rows_per_expert": int(np.diff(row_off).min()),
            "launches": "gate+up: brik_xprep_f16 + brik_gemmg_q4 (grid.z = 2); down: brik_xprep_f16 + brik_gemmg_q4",
            "us_three_calls": round(ms3 * 1e3, 2)}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_baseline(target_s=15.0):
    """JS restatement of the reference CPU matmul (oracle/cpuref.js) on one Qwen3-4B q4 layer set (M=1),
    single-threaded under node, on the headline's own inputs (the same weight tensors and activation
    rows). A first pass times the layer set once and keeps its outputs; the sample then repeats each
    matrix so the whole sample takes about ``target_s`` seconds, and the value is the mean rate.
    Returns (the cpu_baseline object, the reference outputs by shape name) or (None, None)."""
    node = shutil.which("node")
    if node is None:
        return None, None
    from brimkern_amd import synth, layout
    refs = {}

    def run(reps):
        total_ms, nbytes = 0.0, 0
        with tempfile.TemporaryDirectory() as d:
            for si, (name, K, N) in enumerate(QWEN3_4B):
                t = synth.q4_tensor(200 + si, N, K)
                inp, out = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
                with open(inp, "wb") as f:
                    f.write(head_x(K).tobytes())
                    f.write(layout.pack("q4", t).tobytes())
                res = json.loads(subprocess.check_output([node, os.path.join(ROOT, "oracle", "cpuref.js"), "q4", "1",
                                                          str(K), str(N), inp, out, str(reps)]))
                total_ms += res["total_ms"]
                nbytes += reps * (q_bytes("q4", N, K) + 4 * K + 4 * N)
                if name not in refs:
                    refs[name] = np.fromfile(out, np.float32, N)
        return total_ms, nbytes

    t1, _ = run(1)
    reps = max(1, min(200, int(round(target_s * 1e3 / max(t1, 1.0)))))
    total_ms, nbytes = run(reps)
    return ({"value": round(nbytes / (total_ms * 1e-3) / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
             "sample": f"one Qwen3-4B q4 layer set (6 matrices, M=1, {nbytes / reps / 1e6:.1f} MB) x {reps} passes, "
                       f"{total_ms / 1e3:.1f} s, node {subprocess.check_output([node, '--version']).decode().strip()} "
                       f"single-threaded, {cpu_model()}; the headline's inputs"}, refs)


def node_host_timing(timeout=240):
    """The JavaScript host's per-call costs (brimkern_amd/js/host_timing.js under node, a child process
    with its own context): mm, a fused decoder layer's plan runs and an awaited readback op, eager and
    replayed from a recorded graph."""
    node = shutil.which("node")
    if node is None:
        return {"skipped": "node absent"}
    r = subprocess.run([node, os.path.join(ROOT, "brimkern_amd", "js", "host_timing.js")], cwd=ROOT,
                       capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        return {"failed": r.stderr[-500:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


def verify_headline(y_head, refs, layers, tol=1e-5):
    """The headline's last timed step against the CPU reference's outputs on the same inputs: every
    layer's copy of each of the six matrices (all 216 outputs, every row), normwise relative error
    max|y - r| / max|r|. The layer copies hold the same weights, so one reference per shape serves all."""
    if refs is None:
        return {"verified": None, "note": "node absent: no CPU reference outputs"}
    worst, where, off = 0.0, None, 0
    for l in range(layers):
        for name, K, N in QWEN3_4B:
            y, r = y_head[off:off + N], refs[name]
            err = float(np.max(np.abs(y.astype(np.float64) - r)) / max(np.max(np.abs(r)), 1e-30))
            if not np.isfinite(err) or err > worst:
                worst, where = err if np.isfinite(err) else float("inf"), f"layer {l} {name}"
            off += N
    return {"verified": bool(worst <= tol), "max_normwise_rel": worst, "worst": where, "tol": tol,
            "outputs": layers * len(QWEN3_4B),
            "against": "oracle/cpuref.js (the cpu_baseline run) on the same weights and x"}


# ---- HBM traffic of the dominant kernel (two rocprofv3 counter passes in child processes) ---------

CAL_BYTES = 512 << 20      # device-to-device copy of known size: calibrates FETCH_SIZE / WRITE_SIZE


def probe(layers, reps=6):
    """Child-process body of the counter passes: a few plan launches and one calibration copy."""
    from brimkern_amd import Context
    ctx = Context(0)
    plan, bufs = build_layer_plan(ctx, layers)
    for _ in range(reps):
        plan.run()
    ctx.sync()
    a, b = ctx.alloc(CAL_BYTES), ctx.alloc(CAL_BYTES)
    ctx._check(ctx.lib.brik_d2d(ctx.handle, ctx_p(b.ptr), ctx_p(a.ptr), CAL_BYTES))
    ctx.sync()
    print("probe done", flush=True)


def counter_pass(counter, layers, timeout=120):
    """Run the probe under ``rocprofv3 --pmc <counter>``; returns {kernel: [values per dispatch]}."""
    import csv
    import glob
    prof = shutil.which("rocprofv3")
    if prof is None:
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "p", "--",
               sys.executable, os.path.abspath(__file__), "--probe", "--layers", str(layers)]
        env = dict(os.environ, TMPDIR="/tmp")
        r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                           timeout=timeout)
        if r.returncode != 0 or b"probe done" not in r.stdout:
            return None
        out = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for row in csv.DictReader(open(f)):
                if row["Counter_Name"] == counter:
                    out.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return out


def hbm_traffic(layers):
    """HBM bytes per step of the grouped plan: FETCH_SIZE + WRITE_SIZE (KiB per dispatch) of its GEMV
    kernel and of its staging kernel (a large plan stages its distinct input rows in a launch of its
    own), each scaled by what the same counter reads for a device copy of CAL_BYTES."""
    try:
        res = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            vals = counter_pass(counter, layers)
            if not vals:
                return None, None
            gemv = [v for k, vs in vals.items() if k.startswith("brik_gemvg_") for v in vs]
            stage = [v for k, vs in vals.items() if k.startswith("brik_gemv_stage_") for v in vs]
            copy = [v for k, vs in vals.items() if "copyBuffer" in k for v in vs]
            if not gemv or not copy:
                return None, None
            names = [k for k in vals if k.startswith("brik_gemv_stage_")] + [k for k in vals if k.startswith("brik_gemvg_")]
            kernel = " + ".join(names)
            factor = CAL_BYTES / (max(copy) * 1024.0)
            per_step = float(np.median(gemv)) + (float(np.median(stage)) if stage else 0.0)
            res[counter] = (per_step * 1024.0 * factor, factor)
        return {"bytes": res["FETCH_SIZE"][0] + res["WRITE_SIZE"][0],
                "fetch_bytes": round(res["FETCH_SIZE"][0]), "write_bytes": round(res["WRITE_SIZE"][0]),
                "fetch_scale": round(res["FETCH_SIZE"][1], 4), "write_scale": round(res["WRITE_SIZE"][1], 4)}, kernel
    except (subprocess.SubprocessError, OSError, ValueError, KeyError):
        return None, None


def headline_only(ctx, a):
    """The headline plan alone: settle, warmup, timed steps (no per-matrix, small-M or F3 extras)."""
    plan, b = build_layer_plan(ctx, a.layers)
    settle(ctx, lambda i: plan.run(), a.settle)
    ms = time_loop(ctx, lambda i: plan.run(), a.steps, a.warmup)
    plan.destroy()
    for r in b["reps"].values():
        ctx.free(r.buf)
    for bb in (b["xa"], b["xd"], b["ybuf"]):
        ctx.free(bb)
    return {"us": round(ms * 1e3, 2), "GBps": round(b["nbytes"] / (ms * 1e-3) / 1e9, 1)}


def f3_only(ctx, a):
    plan, b = build_layer_plan(ctx, a.layers)
    plan.destroy()
    out = decode_layers_fused(ctx, b["reps"], a.layers, a.steps, a.warmup, not a.no_graph)
    for r in b["reps"].values():
        ctx.free(r.buf)
    for bb in (b["xa"], b["xd"], b["ybuf"]):
        ctx.free(bb)
    return out


def library_gemm_reference(ctx, steps, warmup):
    """A yardstick, not this library's path: hipBLASLt through torch.matmul on the prefill GEMM shape
    (M = 512, K = 2560, N = 9728) with the weights already in f16 / bf16 (3.2x the q4 bytes, nothing
    to dequantize), 8 weight copies rotated (400 MB, past the 256 MB last-level cache), CUDA events on
    torch's stream. torch loads its own HIP runtime, which finds no device once this library's runtime
    holds it, so this runs in a process without a library context."""
    import torch
    M, K, N = 512, 2560, 9728
    g = torch.Generator(device="cuda").manual_seed(0)
    out = {"shape": f"M={M} K={K} N={N}", "library": "hipBLASLt via torch.matmul, x (M, K) @ W.T, W (N, K)"}
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        x = torch.randn(M, K, device="cuda", dtype=dt, generator=g)
        ws = [torch.randn(N, K, device="cuda", dtype=dt, generator=g) * 0.05 for _ in range(8)]
        for i in range(max(warmup, 8)):
            torch.matmul(x, ws[i % 8].t())
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = max(steps, 8)
        a.record()
        for i in range(n):
            torch.matmul(x, ws[i % 8].t())
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / n
        tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
        out[name] = {"us": round(us, 2), "TFLOPs": round(tf, 1), "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
        del x, ws
    torch.cuda.empty_cache()
    return out


ONLY = {
    "headline": headline_only,
    "blasref": lambda ctx, a: library_gemm_reference(ctx, a.steps, a.warmup),
    "f3": f3_only,
    "cfg1": lambda ctx, a: gemv_single_cfg(ctx, "q8", 896, 4864, 600, a.steps, a.warmup),
    "cfg3": lambda ctx, a: gemv_single_cfg(ctx, "q3", 2560, 151936, 700, a.steps, a.warmup),
    "f2": lambda ctx, a: lm_head_topk_cfg3(ctx, a.steps, a.warmup,
                                           gemv_single_cfg(ctx, "q3", 2560, 151936, 700, a.steps, a.warmup)["us"]),
    "cfg4": lambda ctx, a: gemm_cfg4(ctx, a.steps, a.warmup),
    "moe": lambda ctx, a: moe_cfg5(ctx, a.steps, a.warmup),
    "conv": lambda ctx, a: conv_f4(ctx, a.steps, a.warmup),
    "f16w": lambda ctx, a: f16w_f4(ctx, a.steps, a.warmup),
    "f1": lambda ctx, a: quantize_f1(ctx, a.steps, a.warmup),
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed headline steps before the warmup (GPU clock steady state)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 counter passes")
    ap.add_argument("--no-graph", action="store_true",
                    help="no graph replay: time the fused decoder layers and the single-launch lines eagerly "
                         "(rocprofv3's kernel trace has crashed in hipGraphLaunch on the box)")
    ap.add_argument("--only", choices=sorted(ONLY),
                    help="run one workload alone and print its result (for profiler runs; not the bench line)")
    ap.add_argument("--probe", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    global GRAPHS
    GRAPHS = not args.no_graph
    if args.probe:
        probe(args.layers)
        return
    if args.only == "blasref":
        # torch's own HIP runtime must be the first to open the device: no library context here
        log("bench: blasref alone")
        print(json.dumps({"only": args.only, "steps": args.steps, "warmup": args.warmup,
                          "result": library_gemm_reference(None, args.steps, args.warmup)}), flush=True)
        return
    if args.only:
        from brimkern_amd import Context
        ctx = Context(0)
        log(f"bench: {args.only} alone")
        print(json.dumps({"only": args.only, "steps": args.steps, "warmup": args.warmup,
                          "result": ONLY[args.only](ctx, args)}), flush=True)
        ctx.close()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this path has no multi-GPU form in this build (it would shard "
              "the weight rows along N, one slice per GPU, and all-gather y); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    traffic, kernel = (None, None)
    if not args.no_traffic:
        # counter passes run in child processes before this process touches the GPU
        log("bench: HBM traffic counter passes")
        traffic, kernel = hbm_traffic(args.layers)
    from brimkern_amd import Context
    ctx = Context(0)
    log("bench: q4 GEMV layer set")
    ms, nbytes, single, fused, small_m, y_head = gemv_layer_set(ctx, args.steps, args.warmup, args.layers,
                                                                args.settle, not args.no_graph)
    value = nbytes / (ms * 1e-3) / 1e9
    extra = {"per_matrix_single_launch": single, "f3_decode_layers_fused_qwen3_4b": fused,
             "small_m_qwen3_4b": dict(small_m, note="matmul_t_q4 at M rows per call (the reference's "
                                      "matmul_t_q4_tiled range 2 <= M < 16): the routed path (auto), the GEMV "
                                      "re-streaming W per row, the tiled MFMA GEMM and the split-K MFMA GEMM, "
                                      "graph-replayed; weight_GBps = W bytes (read once) / auto time")}
    if not args.no_extra:
        log("bench: q8 / q3 small-M")
        extra["small_m_q8_q3_qwen3_4b"] = small_m_formats(ctx)
        log("bench: cfg1 q8 GEMV")
        extra["cfg1_q8_gemv_K896_N4864"] = gemv_single_cfg(ctx, "q8", 896, 4864, 600, args.steps, args.warmup)
        log("bench: cfg3 q3 LM head")
        extra["cfg3_q3_gemv_K2560_N151936"] = gemv_single_cfg(ctx, "q3", 2560, 151936, 700, args.steps, args.warmup)
        log("bench: cfg3 LM head + sampling pre-work")
        extra["f2_lm_head_topk_q3_K2560_N151936"] = lm_head_topk_cfg3(
            ctx, args.steps, args.warmup, extra["cfg3_q3_gemv_K2560_N151936"]["us"])
        log("bench: cfg4 q4 GEMM")
        extra["cfg4_q4_gemm_M512_K2560_N9728"] = gemm_cfg4(ctx, args.steps, args.warmup)
        log("bench: cfg5 MoE")
        extra["cfg5_moe_q4_gate_up_down"] = moe_cfg5(ctx, args.steps, args.warmup)
        log("bench: F4 q4 convolution")
        extra["f4_conv2d_q4_320x64x64_k3"] = conv_f4(ctx, args.steps, args.warmup)
        log("bench: F4 f16-weight matmul")
        extra["f4_matmul_t_f16w_K2560_N9728"] = f16w_f4(ctx, args.steps, args.warmup)
        log("bench: F1 encoders")
        extra["f1_quantize_f32_to_planes_N9728_K2560"] = quantize_f1(ctx, args.steps, args.warmup)
        log("bench: JS host (node) per-call costs")
        extra["js_host_node"] = node_host_timing()
    cpu, refs = (None, None) if args.no_cpu else cpu_baseline()
    check = verify_headline(y_head, refs, args.layers) if not args.no_cpu else {"verified": None,
                                                                               "note": "--no-cpu"}
    line = {
        "metric": "q4 GEMV HBM GB/s (% of peak) at Qwen3-4B shapes; prefill q4 GEMM TFLOP/s",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "settle_s": args.settle, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32", "x_staging": "per 32-element group as 24-bit block floating point (exact int32 dot "
                                     "products with the codes, one f32 rescale per group), f32 accumulation",
        "data": "synthetic (seeded SplitMix64), random q4 weights of the Qwen3-4B shapes",
        "verified": check.get("verified"), "verification": check,
        "config": {"workload": f"matmul_t_q4 decode GEMV, Qwen3-4B layer set x {args.layers} layers "
                               f"(216 matrices, M=1), grouped plan: one staging + one GEMV launch per step",
                   "bytes_per_step": nbytes, "layers": args.layers},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else round(traffic["bytes"]),
                     "traffic_detail": traffic, "algorithmic_bytes": nbytes,
                     "kernel": kernel or "brik_gemv_stage_q4 + brik_gemvg_q4 (grouped plan)",
                     "us_per_launch": round(ms * 1e3, 2)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
