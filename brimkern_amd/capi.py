"""ctypes binding of ``libbrik.so`` (the C ABI in ``include/brik.h``).

This is the Python-side host of the drop-in boundary (tests, bench, smoke); the JavaScript host is
``brimkern_amd/js`` over the N-API addon. Both call the same C entry points. Nothing here falls
back to CPU: if the library is missing or no gfx950 device is present, construction raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libbrik.so")

BRIK_OK, BRIK_EINVAL, BRIK_EALIGN, BRIK_EHIP, BRIK_ENOMEM, BRIK_ENODEV, BRIK_EMODULE = 0, -1, -2, -3, -4, -5, -6
BRIK_EVALID = -7
BRIK_OPT_PATH, BRIK_OPT_GEMV_VARIANT = 1, 2
BRIK_GEMV_VARIANTS = 11
BRIK_OPT_GEMM_TILE, BRIK_GEMM_TILES = 3, 23
BRIK_OPT_PLAN_STAGE, BRIK_OPT_PLAN_SETS, BRIK_OPT_SPLITK, BRIK_OPT_GEMV_BLOCKS = 4, 5, 6, 7
PATH_AUTO, PATH_GEMV, PATH_GEMM = 0, 1, 2
BRIK_PATH_GEMV, BRIK_PATH_GEMV_STAGED, BRIK_PATH_TILED, BRIK_PATH_SPLITK = 1, 2, 3, 4

# every exported symbol of include/brik.h with (restype, argtypes)
_P, _I, _Z, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.POINTER(ctypes.c_float)
SIGNATURES = {
    "brik_create": (_I, [_I, ctypes.POINTER(_P)]),
    "brik_destroy": (None, [_P]),
    "brik_last_error": (ctypes.c_char_p, [_P]),
    "brik_last_path": (_I, [_P]),
    "brik_strerror": (ctypes.c_char_p, [_I]),
    "brik_device_count": (_I, [ctypes.POINTER(_I)]),
    "brik_alloc": (_I, [_P, _Z, ctypes.POINTER(_P)]),
    "brik_free": (_I, [_P, _P]),
    "brik_h2d": (_I, [_P, _P, _P, _Z]),
    "brik_d2h": (_I, [_P, _P, _P, _Z]),
    "brik_d2d": (_I, [_P, _P, _P, _Z]),
    "brik_h2d_async": (_I, [_P, _P, _P, _Z]),
    "brik_sync": (_I, [_P]),
    "brik_fence_record": (_I, [_P, ctypes.POINTER(_P)]),
    "brik_fence_d2h": (_I, [_P, _P, _P, _Z]),
    "brik_fence_error": (ctypes.c_char_p, [_P]),
    "brik_fence_destroy": (None, [_P]),
    "brik_self_validate": (_I, [_P, ctypes.c_char_p, _Z]),
    "brik_matmul_t_q8": (_I, [_P, _P, _P, _P, _P, _I, _I, _I]),
    "brik_matmul_t_q4": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "brik_matmul_t_q3": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "brik_matmul_t_q4_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "brik_moe_matmul_t_q4": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "brik_moe_matmul_t_q4_x2": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "brik_dequant_q8_f32": (_I, [_P, _P, _P, _P, _Z]),
    "brik_dequant_q4_f32": (_I, [_P, _P, _P, _P, _P, _Z]),
    "brik_dequant_q3_f32": (_I, [_P, _P, _P, _P, _P, _P, _Z]),
    "brik_quantize_q8": (_I, [_P, _P, _P, _P, _Z]),
    "brik_quantize_q4": (_I, [_P, _P, _P, _P, _P, _Z]),
    "brik_quantize_q3": (_I, [_P, _P, _P, _P, _P, _P, _Z]),
    "brik_f16_to_f32": (_I, [_P, _P, _P, _Z]),
    "brik_matmul_t_f16w": (_I, [_P, _P, _P, _P, _I, _I, _I]),
    "brik_conv2d_q8": (_I, [_P, _P, _P, _P, _P, _P] + [_I] * 8),
    "brik_conv2d_q4": (_I, [_P, _P, _P, _P, _P, _P, _P] + [_I] * 8),
    "brik_timer_begin": (_I, [_P]),
    "brik_timer_end": (_I, [_P, _F]),
    "brik_set_option": (_I, [_P, _I, _I]),
    "brik_gemv_plan_create": (_I, [_P, _I, _P, _I, ctypes.POINTER(_P)]),
    "brik_gemv_plan_run": (_I, [_P, _P]),
    "brik_gemv_plan_destroy": (None, [_P, _P]),
    "brik_gemv_plan_create_ex": (_I, [_P, _I, _P, _I, ctypes.POINTER(_P)]),
    "brik_gemv_plan_create_glu": (_I, [_P, _I, _P, _P, _P, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "brik_graph_begin": (_I, [_P]),
    "brik_graph_end": (_I, [_P, ctypes.POINTER(_P)]),
    "brik_graph_launch": (_I, [_P, _P]),
    "brik_graph_destroy": (None, [_P, _P]),
    "brik_logits_topk": (_I, [_P, _P, _I, _P, _I, ctypes.c_float, ctypes.c_float, _I, _P, _P]),
    "brik_lm_head_topk_q8": (_I, [_P, _P, _P, _P, _I, _I, _P, _I, ctypes.c_float, ctypes.c_float, _I, _P, _P]),
    "brik_lm_head_topk_q4": (_I, [_P, _P, _P, _P, _P, _I, _I, _P, _I, ctypes.c_float, ctypes.c_float, _I, _P, _P]),
    "brik_lm_head_topk_q3": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _P, _I, ctypes.c_float, ctypes.c_float, _I, _P,
                                  _P]),
}
BRIK_TOPK_MAX = 64
BRIK_NOALLOC_SCRATCH_BYTES = 16 << 20
BRIK_STAGING_RING_BYTES = 32 << 20

FMT_CODES = {"q8": 8, "q4": 4, "q3": 3}


class GemvJob(ctypes.Structure):
    """``brik_gemv_job`` of include/brik.h."""
    _fields_ = [("x", _P), ("p0", _P), ("p1", _P), ("scales", _P), ("mins", _P), ("y", _P),
                ("K", ctypes.c_int32), ("N", ctypes.c_int32)]


class GemvJobEx(ctypes.Structure):
    """``brik_gemv_job_ex`` of include/brik.h (fused input transform and residual)."""
    _fields_ = [("job", GemvJob), ("gate", _P), ("norm_w", _P), ("res", _P), ("eps", ctypes.c_float),
                ("flags", ctypes.c_int32)]


BRIK_JOB_GAIN_ONE_PLUS, BRIK_JOB_ACT_GELU = 1, 2


class BrikError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"brik error {code}: {msg}")
        self.code = code


_lib = None


def load_library(path: str = LIB_PATH):
    """Load libbrik.so and declare every entry point. Raises if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing: run `python -m brimkern_amd.build` (no CPU fallback exists)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def device_count() -> int:
    n = ctypes.c_int(0)
    load_library().brik_device_count(ctypes.byref(n))
    return n.value


class DeviceBuffer:
    """A device allocation owned by a :class:`Context`."""

    __slots__ = ("ctx", "ptr", "nbytes")

    def __init__(self, ctx: "Context", ptr: int, nbytes: int):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes

    def offset(self, nbytes: int) -> int:
        """Raw device address ``nbytes`` into the buffer (for plane views into a packed blob)."""
        assert 0 <= nbytes <= self.nbytes
        return self.ptr + nbytes

    def free(self):
        if self.ptr:
            self.ctx._check(self.ctx.lib.brik_free(self.ctx.handle, _P(self.ptr)))
            self.ptr = 0

    def __int__(self):
        return self.ptr


def _addr(p) -> _P:
    if p is None:
        return _P(None)
    if isinstance(p, DeviceBuffer):
        return _P(p.ptr)
    return _P(int(p))


class Context:
    """One device + one stream (``brik_ctx``)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _P()
        rc = self.lib.brik_create(device, ctypes.byref(h))
        if rc != BRIK_OK:
            raise BrikError(rc, f"brik_create({device}): {self.lib.brik_strerror(rc).decode()}")
        self.handle = h
        self._buffers = []

    def _check(self, rc: int):
        if rc != BRIK_OK:
            raise BrikError(rc, self.lib.brik_last_error(self.handle).decode())
        return rc

    def close(self):
        if getattr(self, "handle", None):
            for b in self._buffers:
                b.free()
            self._buffers.clear()
            self.lib.brik_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- memory -----------------------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        p = _P()
        self._check(self.lib.brik_alloc(self.handle, max(int(nbytes), 1), ctypes.byref(p)))
        b = DeviceBuffer(self, p.value, int(nbytes))
        self._buffers.append(b)
        return b

    def free(self, buf: DeviceBuffer):
        buf.free()
        if buf in self._buffers:
            self._buffers.remove(buf)

    def upload(self, arr: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        b = self.alloc(a.nbytes)
        self.h2d(b, a)
        return b

    def h2d(self, dst, arr: np.ndarray, dst_offset: int = 0):
        a = np.ascontiguousarray(arr)
        self._check(self.lib.brik_h2d(self.handle, _P(int(_addr(dst).value or 0) + dst_offset),
                                      _P(a.ctypes.data), a.nbytes))

    def h2d_async(self, dst, arr: np.ndarray, dst_offset: int = 0):
        """Upload without waiting for earlier work (brik_h2d_async): ``arr`` may change on return."""
        a = np.ascontiguousarray(arr)
        self._check(self.lib.brik_h2d_async(self.handle, _P(int(_addr(dst).value or 0) + dst_offset),
                                            _P(a.ctypes.data), a.nbytes))

    def download(self, src, dtype, count: int, src_offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        self._check(self.lib.brik_d2h(self.handle, _P(out.ctypes.data),
                                      _P(int(_addr(src).value or 0) + src_offset), out.nbytes))
        return out

    def sync(self):
        self._check(self.lib.brik_sync(self.handle))

    def fence(self) -> "Fence":
        """Mark the current end of the stream (brik_fence_record)."""
        h = _P()
        self._check(self.lib.brik_fence_record(self.handle, ctypes.byref(h)))
        return Fence(self, h)

    def self_validate(self):
        """The load-time kernel checks (brik_self_validate): returns None when every check passes, else
        the name of the first failing check (BRIK_EVALID); other errors raise."""
        buf = ctypes.create_string_buffer(64)
        rc = self.lib.brik_self_validate(self.handle, buf, 64)
        if rc == BRIK_EVALID:
            return buf.value.decode()
        self._check(rc)
        return None

    def set_option(self, key: int, value: int):
        self._check(self.lib.brik_set_option(self.handle, key, value))

    def last_path(self) -> int:
        """BRIK_PATH_* of the last matmul call on this context (0 before any, or for K = 0)."""
        return self.lib.brik_last_path(self.handle)

    def timer_begin(self):
        self._check(self.lib.brik_timer_begin(self.handle))

    def timer_end(self) -> float:
        ms = ctypes.c_float(0)
        self._check(self.lib.brik_timer_end(self.handle, ctypes.byref(ms)))
        return ms.value

    # ---- compute (device pointers, enqueue only) -------------------------------------------
    def matmul_t_q8(self, x, codes, sc, y, M, K, N):
        self._check(self.lib.brik_matmul_t_q8(self.handle, _addr(x), _addr(codes), _addr(sc), _addr(y), M, K, N))

    def matmul_t_q4(self, x, nib, sc, mn, y, M, K, N):
        self._check(self.lib.brik_matmul_t_q4(self.handle, _addr(x), _addr(nib), _addr(sc), _addr(mn),
                                              _addr(y), M, K, N))

    def matmul_t_q4_noalloc(self, x, nib, sc, mn, y, M, K, N):
        """:meth:`matmul_t_q4` on the library's fixed per-device scratch: no device allocation."""
        self._check(self.lib.brik_matmul_t_q4_noalloc(self.handle, _addr(x), _addr(nib), _addr(sc), _addr(mn),
                                                      _addr(y), M, K, N))

    def matmul_t_q3(self, x, lo, hi, sc, mn, y, M, K, N):
        self._check(self.lib.brik_matmul_t_q3(self.handle, _addr(x), _addr(lo), _addr(hi), _addr(sc),
                                              _addr(mn), _addr(y), M, K, N))

    def moe_matmul_t_q4(self, x, row_off, nib, sc, mn, y, E, R, K, N):
        self._check(self.lib.brik_moe_matmul_t_q4(self.handle, _addr(x), _addr(row_off), _addr(nib),
                                                  _addr(sc), _addr(mn), _addr(y), E, R, K, N))

    def moe_matmul_t_q4_x2(self, x, row_off, a, y_a, b, y_b, E, R, K, N):
        """Two stacked q4 tensors (``a``, ``b``: (nib, sc, mn) address triples) on the same routed rows,
        one launch (brik_moe_matmul_t_q4_x2)."""
        self._check(self.lib.brik_moe_matmul_t_q4_x2(self.handle, _addr(x), _addr(row_off), *map(_addr, a),
                                                     _addr(y_a), *map(_addr, b), _addr(y_b), E, R, K, N))

    def gemv_plan(self, fmt: str, jobs) -> "GemvPlan":
        """jobs: iterable of dicts with x, p0, p1, sc, mn, y (device addresses), K, N, and optionally the
        fusions of ``brik_gemv_job_ex``: gate, norm_w, eps, one_plus, gelu, res. Jobs without any
        fusion key go through ``brik_gemv_plan_create``, the others through the ``_ex`` form."""
        jobs = list(jobs)
        fused = any(k in j for j in jobs for k in ("gate", "norm_w", "res"))
        h = _P()
        if not fused:
            arr = (GemvJob * len(jobs))()
            for i, j in enumerate(jobs):
                arr[i] = GemvJob(_addr(j["x"]), _addr(j["p0"]), _addr(j.get("p1")), _addr(j["sc"]),
                                 _addr(j.get("mn")), _addr(j["y"]), j["K"], j["N"])
            self._check(self.lib.brik_gemv_plan_create(self.handle, FMT_CODES[fmt], ctypes.cast(arr, _P), len(jobs),
                                                       ctypes.byref(h)))
            return GemvPlan(self, h)
        arr = (GemvJobEx * len(jobs))()
        for i, j in enumerate(jobs):
            arr[i] = _job_ex(j)
        self._check(self.lib.brik_gemv_plan_create_ex(self.handle, FMT_CODES[fmt], ctypes.cast(arr, _P), len(jobs),
                                                      ctypes.byref(h)))
        return GemvPlan(self, h)

    def gemv_plan_glu(self, fmt: str, gate, up, down):
        """The linked (gate/up, down) plans of ``brik_gemv_plan_create_glu``; each job a dict as for
        :meth:`gemv_plan`. down must read gate's and up's outputs (``gate=gate["y"]``, ``x=up["y"]``).
        Returns ``(gate_up_plan, down_plan)``; run them in that order."""
        jobs = (GemvJobEx * 3)(_job_ex(gate), _job_ex(up), _job_ex(down))
        hg, hd = _P(), _P()
        base = ctypes.addressof(jobs)
        size = ctypes.sizeof(GemvJobEx)
        self._check(self.lib.brik_gemv_plan_create_glu(self.handle, FMT_CODES[fmt], _P(base), _P(base + size),
                                                       _P(base + 2 * size), ctypes.byref(hg), ctypes.byref(hd)))
        return GemvPlan(self, hg), GemvPlan(self, hd)

    # ---- recorded launches (HIP graphs) ---------------------------------------------------------
    def graph_begin(self):
        """Record (not run) every launch enqueued from now on until :meth:`graph_end`."""
        self._check(self.lib.brik_graph_begin(self.handle))

    def graph_end(self) -> "Graph":
        h = _P()
        self._check(self.lib.brik_graph_end(self.handle, ctypes.byref(h)))
        return Graph(self, h)

    # ---- sampling pre-work ----------------------------------------------------------------
    def logits_topk(self, logits, n, recent, n_recent, penalty, softcap, k, ids, vals):
        """Softcap, repetition penalty (in place on ``logits``) and the top ``k``, on the stream."""
        self._check(self.lib.brik_logits_topk(self.handle, _addr(logits), n, _addr(recent), n_recent, penalty,
                                              softcap, k, _addr(ids), _addr(vals)))

    def lm_head_topk(self, fmt: str, x, planes, K, vocab, recent, n_recent, penalty, softcap, k, ids, vals):
        """``x . deq(W)^T`` over the vocab, then :meth:`logits_topk` on the logits (a workspace)."""
        tail = (K, vocab, _addr(recent), n_recent, penalty, softcap, k, _addr(ids), _addr(vals))
        fn = getattr(self.lib, f"brik_lm_head_topk_{fmt}")
        self._check(fn(self.handle, _addr(x), *[_addr(p) for p in planes], *tail))

    def dequant_q8(self, codes, sc, out, n):
        self._check(self.lib.brik_dequant_q8_f32(self.handle, _addr(codes), _addr(sc), _addr(out), n))

    def dequant_q4(self, nib, sc, mn, out, n):
        self._check(self.lib.brik_dequant_q4_f32(self.handle, _addr(nib), _addr(sc), _addr(mn), _addr(out), n))

    def dequant_q3(self, lo, hi, sc, mn, out, n):
        self._check(self.lib.brik_dequant_q3_f32(self.handle, _addr(lo), _addr(hi), _addr(sc), _addr(mn),
                                                 _addr(out), n))

    def quantize(self, fmt: str, src, planes, n):
        """Encode ``n`` f32 values at ``src`` into the planes of ``fmt`` (the unpackQ* order:
        q8 codes, sc; q4 nib, sc, mn; q3 lo, hi, sc, mn), byte-identical to quantizeQ*."""
        fn = getattr(self.lib, f"brik_quantize_{fmt}")
        self._check(fn(self.handle, _addr(src), *[_addr(p) for p in planes], n))

    def conv2d(self, fmt: str, inp, planes, bias, out, Cin, H, W, Cout, kh, kw, stride=1, pad=0):
        """conv2d_direct_q8 / _q4: ``out[Cout, OH, OW]`` from ``inp[Cin, H, W]`` and a q8 (codes, sc) or
        q4 (nib, sc, mn) OIHW weight; ``bias`` may be None."""
        fn = getattr(self.lib, f"brik_conv2d_{fmt}")
        self._check(fn(self.handle, _addr(inp), *[_addr(p) for p in planes], _addr(bias), _addr(out),
                       Cin, H, W, Cout, kh, kw, stride, pad))

    def matmul_t_f16w(self, x, w, y, M, K, N):
        """y = x . W^T with W [N, K] IEEE f16 bits (MATMUL_T_F16W)."""
        self._check(self.lib.brik_matmul_t_f16w(self.handle, _addr(x), _addr(w), _addr(y), M, K, N))

    def f16_to_f32(self, src, out, n):
        self._check(self.lib.brik_f16_to_f32(self.handle, _addr(src), _addr(out), n))


class Fence:
    """A point on the context stream (``brik_fence``): :meth:`d2h` waits for it, then copies to host;
    safe to call from another thread while the context keeps enqueueing."""

    def __init__(self, ctx: Context, handle):
        self.ctx, self.handle = ctx, handle

    def d2h(self, src, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        rc = self.ctx.lib.brik_fence_d2h(self.handle, _P(out.ctypes.data), _addr(src), out.nbytes)
        if rc != BRIK_OK:
            raise BrikError(rc, self.ctx.lib.brik_fence_error(self.handle).decode())
        return out

    def destroy(self):
        if self.handle:
            self.ctx.lib.brik_fence_destroy(self.handle)
            self.handle = None


class Graph:
    """A recorded launch sequence (``brik_graph``): :meth:`launch` replays it on the context stream."""

    def __init__(self, ctx: Context, handle):
        self.ctx, self.handle = ctx, handle

    def launch(self):
        self.ctx._check(self.ctx.lib.brik_graph_launch(self.ctx.handle, self.handle))

    def destroy(self):
        if self.handle:
            self.ctx.lib.brik_graph_destroy(self.ctx.handle, self.handle)
            self.handle = None


def _job_ex(j) -> GemvJobEx:
    base = GemvJob(_addr(j["x"]), _addr(j["p0"]), _addr(j.get("p1")), _addr(j["sc"]), _addr(j.get("mn")),
                   _addr(j["y"]), j["K"], j["N"])
    flags = (BRIK_JOB_GAIN_ONE_PLUS if j.get("one_plus") else 0) | (BRIK_JOB_ACT_GELU if j.get("gelu") else 0)
    return GemvJobEx(base, _addr(j.get("gate")), _addr(j.get("norm_w")), _addr(j.get("res")),
                     float(j.get("eps", 1e-6)), flags)


class GemvPlan:
    def __init__(self, ctx: Context, handle):
        self.ctx, self.handle = ctx, handle

    def run(self):
        self.ctx._check(self.ctx.lib.brik_gemv_plan_run(self.ctx.handle, self.handle))

    def destroy(self):
        if self.handle:
            self.ctx.lib.brik_gemv_plan_destroy(self.ctx.handle, self.handle)
            self.handle = None
