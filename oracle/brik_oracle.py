"""Python face of the CPU oracle (TEST INFRASTRUCTURE ONLY — the checker, never the product).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module.

Two parts:

* ctypes wrappers over ``brik_oracle.c`` — the C restatement of the reference's CPU arithmetic:
  f16 decode/encode (``src/lib/brik/f16.ts:8-34``), ``dequantizeQ8/Q4/Q3``
  (``src/lib/brik/q8web.ts:74-83``, ``q4web.ts:82-96``, ``q3web.ts:97-110``) and the
  self-validation reference matmul (``src/lib/webgpu/kernels.ts:2335-2337``: dequantize to
  Float32Array, sum ``a*w`` left to right in a JS double, round once to f32).
* numpy restatements of the reference's encoder side, used only to re-derive the reference's own
  codec unit tests as pins of the layout: ``quantizeQ8/Q4/Q3`` (``q8web.ts:28-50``,
  ``q4web.ts:28-53``, ``q3web.ts:34-60``), ``packQ*`` / ``unpackQ*`` offsets
  (``q8web.ts:55-72``, ``q4web.ts:58-80``, ``q3web.ts:65-95``) and the byte-length formulas
  (``q8web.ts:23-26``, ``q4web.ts:23-26``, ``q3web.ts:29-32``).

Pinning status (which independent check fixes each function) is listed in the test files
``tests/test_oracle_*.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

GROUP = 32
_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")
_SRC = os.path.join(_HERE, "brik_oracle.c")

__all__ = [
    "GROUP", "build_oracle", "f16_to_f64", "f32_to_f16",
    "dequant_q8", "dequant_q4", "dequant_q3",
    "matmul_t_q8", "matmul_t_q4", "matmul_t_q3", "moe_matmul_t_q4",
    "quantize_q8", "quantize_q4", "quantize_q3",
    "pack_q8", "pack_q4", "pack_q3", "unpack_q8", "unpack_q4", "unpack_q3",
    "q8_byte_length", "q4_byte_length", "q3_byte_length", "js_round",
    "softcap_logits", "penalize_logits", "top_k",
    "rmsnorm", "swiglu", "geglu", "conv2d", "matmul_t_f16w",
]


def build_oracle(force: bool = False) -> str:
    """Compile ``brik_oracle.c`` into ``oracle/liboracle.so`` (gcc, OpenMP, no FP contraction)."""
    if force or not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(_SRC):
        cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
               "-fno-fast-math", "-Wall", "-o", _SO + ".tmp", _SRC, "-lm"]
        subprocess.check_call(cmd)
        os.replace(_SO + ".tmp", _SO)
    return _SO


_lib = None


def _L():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(build_oracle())
        P = ctypes.c_void_p
        I = ctypes.c_int
        Z = ctypes.c_size_t
        lib.oracle_f16_to_f64_n.argtypes = [P, Z, P]
        lib.oracle_f32_to_f16_n.argtypes = [P, Z, P]
        lib.oracle_dequant_q8.argtypes = [P, P, Z, P]
        lib.oracle_dequant_q4.argtypes = [P, P, P, Z, P]
        lib.oracle_dequant_q3.argtypes = [P, P, P, P, Z, P]
        lib.oracle_matmul_t_q8.argtypes = [P, P, P, I, I, I, P, P, I]
        lib.oracle_matmul_t_q4.argtypes = [P, P, P, P, I, I, I, P, P, I]
        lib.oracle_matmul_t_q3.argtypes = [P, P, P, P, P, I, I, I, P, P, I]
        lib.oracle_moe_matmul_t_q4.argtypes = [P, P, P, P, P, I, I, I, P, I]
        lib.oracle_conv2d.argtypes = [P, P, P, I, I, I, I, I, I, I, I, P, P]
        _lib = lib
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- f16 (f16.ts) ------------------------------------------------------------------------

def f16_to_f64(h) -> np.ndarray:
    """``f16BitsToF32`` (f16.ts:25-34): the JS double it returns, per element."""
    h = _c(h, np.uint16).ravel()
    out = np.empty(h.size, np.float64)
    _L().oracle_f16_to_f64_n(_p(h), h.size, _p(out))
    return out


def f32_to_f16(v) -> np.ndarray:
    """``f32ToF16Bits`` (f16.ts:8-22): RNE, flush below 2^-14, clamp to 0x7bff."""
    v = _c(v, np.float32).ravel()
    out = np.empty(v.size, np.uint16)
    _L().oracle_f32_to_f16_n(_p(v), v.size, _p(out))
    return out


# ---- dequant (q*web.ts) ------------------------------------------------------------------

def dequant_q8(codes, sc) -> np.ndarray:
    codes = _c(codes, np.int8).ravel(); sc = _c(sc, np.uint16).ravel()
    assert codes.size == sc.size * GROUP
    out = np.empty(codes.size, np.float32)
    _L().oracle_dequant_q8(_p(codes), _p(sc), codes.size, _p(out))
    return out


def dequant_q4(nib, sc, mn) -> np.ndarray:
    nib = _c(nib, np.uint8).ravel(); sc = _c(sc, np.uint16).ravel(); mn = _c(mn, np.uint16).ravel()
    n = nib.size * 2
    assert sc.size * GROUP == n and mn.size == sc.size
    out = np.empty(n, np.float32)
    _L().oracle_dequant_q4(_p(nib), _p(sc), _p(mn), n, _p(out))
    return out


def dequant_q3(lo, hi, sc, mn) -> np.ndarray:
    lo = _c(lo, np.uint32).ravel(); hi = _c(hi, np.uint32).ravel()
    sc = _c(sc, np.uint16).ravel(); mn = _c(mn, np.uint16).ravel()
    n = lo.size * 16
    assert hi.size * 32 == n and sc.size * GROUP == n and mn.size == sc.size
    out = np.empty(n, np.float32)
    _L().oracle_dequant_q3(_p(lo), _p(hi), _p(sc), _p(mn), n, _p(out))
    return out


# ---- reference matmul (kernels.ts:2335-2337) -------------------------------------------

def _mm_out(M, N, want_den):
    y = np.empty((M, N), np.float32)
    den = np.empty((M, N), np.float64) if want_den else None
    return y, den


def matmul_t_q8(x, codes, sc, M, K, N, absden=False, threads=0):
    x = _c(x, np.float32); codes = _c(codes, np.int8); sc = _c(sc, np.uint16)
    assert x.size == M * K and codes.size == N * K and sc.size == N * K // GROUP and K % GROUP == 0
    y, den = _mm_out(M, N, absden)
    _L().oracle_matmul_t_q8(_p(x), _p(codes), _p(sc), M, K, N, _p(y), _p(den), threads)
    return (y, den) if absden else y


def matmul_t_q4(x, nib, sc, mn, M, K, N, absden=False, threads=0):
    x = _c(x, np.float32); nib = _c(nib, np.uint8); sc = _c(sc, np.uint16); mn = _c(mn, np.uint16)
    assert x.size == M * K and nib.size * 2 == N * K and sc.size == N * K // GROUP and K % GROUP == 0
    y, den = _mm_out(M, N, absden)
    _L().oracle_matmul_t_q4(_p(x), _p(nib), _p(sc), _p(mn), M, K, N, _p(y), _p(den), threads)
    return (y, den) if absden else y


def matmul_t_q3(x, lo, hi, sc, mn, M, K, N, absden=False, threads=0):
    x = _c(x, np.float32); lo = _c(lo, np.uint32); hi = _c(hi, np.uint32)
    sc = _c(sc, np.uint16); mn = _c(mn, np.uint16)
    assert x.size == M * K and lo.size * 16 == N * K and hi.size * 32 == N * K and K % GROUP == 0
    y, den = _mm_out(M, N, absden)
    _L().oracle_matmul_t_q3(_p(x), _p(lo), _p(hi), _p(sc), _p(mn), M, K, N, _p(y), _p(den), threads)
    return (y, den) if absden else y


def moe_matmul_t_q4(x_sorted, row_off, nib, sc, mn, E, K, N, threads=0):
    """Reference matmul applied per expert over a stacked [E, N, K] q4 tensor (no reference
    counterpart exists; the per-expert arithmetic is kernels.ts:2335-2337)."""
    x = _c(x_sorted, np.float32); ro = _c(row_off, np.int32)
    nib = _c(nib, np.uint8); sc = _c(sc, np.uint16); mn = _c(mn, np.uint16)
    R = int(ro[E])
    assert ro.size == E + 1 and x.size == R * K and nib.size * 2 == E * N * K
    y = np.zeros((R, N), np.float32)
    _L().oracle_moe_matmul_t_q4(_p(x), _p(ro), _p(nib), _p(sc), _p(mn), E, K, N, _p(y), threads)
    return y


# ---- encoder side, numpy (used to re-derive the reference's codec tests) ---------------

def js_round(v: np.ndarray) -> np.ndarray:
    """``Math.round``: nearest integer, ties toward +infinity (exact for doubles)."""
    v = np.asarray(v, np.float64)
    f = np.floor(v)
    return f + ((v - f) >= 0.5)


def q8_byte_length(n: int) -> int:   # q8web.ts:23-26
    return n + (n // GROUP) * 2


def q4_byte_length(n: int) -> int:   # q4web.ts:23-26
    g = n // GROUP
    return n // 2 + g * 2 + g * 2


def q3_byte_length(n: int) -> int:   # q3web.ts:29-32
    g = n // GROUP
    return (n // 16) * 4 + (n // 32) * 4 + g * 2 + g * 2


def _groups(data):
    d = np.asarray(data, np.float32).astype(np.float64)
    if d.size % GROUP:
        raise ValueError(f"length {d.size} not a multiple of {GROUP}")
    return d.reshape(-1, GROUP)


def _or_tiny(v):
    """``x || 1e-8`` for a JS number: 0 and NaN are falsy."""
    v = np.asarray(v, np.float64)
    return np.where((v == 0) | np.isnan(v), 1e-8, v)


def _first_equal(d, v):
    """Per row, the first element of ``d`` equal to ``v`` (keeps the sign of a zero), else ``v``."""
    hit = d == v[:, None]
    first = d[np.arange(d.shape[0]), hit.argmax(axis=1)]
    return np.where(hit.any(axis=1), first, v)


def _store_code(q):
    """A clamped code as a typed-array store keeps it: NaN (from a NaN input) becomes 0."""
    return np.where(np.isnan(q), 0.0, q)


def quantize_q8(data):
    """``quantizeQ8`` (q8web.ts:28-50). Returns (codes int8[n], scales u16[n/32])."""
    d = _groups(data)
    # the reference's loop: `if (a > amax) amax = a` from 0, so NaN never wins
    amax = np.fmax.reduce(np.abs(d), axis=1, initial=0.0)
    with np.errstate(over="ignore", invalid="ignore"):
        scale = _or_tiny(amax / 127)
        sH = f32_to_f16(scale.astype(np.float32))
        s = _or_tiny(f16_to_f64(sH))
        q = _store_code(np.clip(js_round(d / s[:, None]), -127, 127))
    return q.astype(np.int8).ravel(), sH


def _quant_asym(data, levels):
    d = _groups(data)
    # `if (v < mn) mn = v; if (v > mx) mx = v` from +-Infinity: NaN is skipped, an all-NaN group
    # keeps mn = Infinity, mx = -Infinity, and among equal values (+0 and -0) the first one stays
    mn = _first_equal(d, np.fmin.reduce(d, axis=1, initial=np.inf))
    mx = _first_equal(d, np.fmax.reduce(d, axis=1, initial=-np.inf))
    with np.errstate(over="ignore", invalid="ignore"):
        scale = _or_tiny((mx - mn) / levels)
        sH = f32_to_f16(scale.astype(np.float32))
        mH = f32_to_f16(mn.astype(np.float32))
        s = _or_tiny(f16_to_f64(sH))
        m = f16_to_f64(mH)
        q = _store_code(np.clip(js_round((d - m[:, None]) / s[:, None]), 0, levels)).astype(np.uint32).ravel()
    return q, sH, mH


def quantize_q4(data):
    """``quantizeQ4`` (q4web.ts:28-53). Returns (nibbles u8[n/2], scales, mins)."""
    q, sH, mH = _quant_asym(data, 15)
    nib = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)   # low nibble = even index
    return nib, sH, mH


def quantize_q3(data):
    """``quantizeQ3`` (q3web.ts:34-60). Returns (lo u32[n/16], hi u32[n/32], scales, mins)."""
    q, sH, mH = _quant_asym(data, 7)
    n = q.size
    idx = np.arange(n, dtype=np.uint64)
    lo = np.zeros(n // 16, np.uint64)
    hi = np.zeros(n // 32, np.uint64)
    np.bitwise_or.at(lo, (idx >> 4).astype(np.int64), ((q & 3).astype(np.uint64) << ((idx & 15) * 2)))
    np.bitwise_or.at(hi, (idx >> 5).astype(np.int64), ((q >> 2).astype(np.uint64) << (idx & 31)))
    return lo.astype(np.uint32), hi.astype(np.uint32), sH, mH


def pack_q8(codes, sc) -> np.ndarray:
    """``packQ8`` (q8web.ts:55-62): [codes | scales LE]."""
    return np.concatenate([_c(codes, np.int8).view(np.uint8), _c(sc, "<u2").view(np.uint8)])


def pack_q4(nib, sc, mn) -> np.ndarray:
    """``packQ4`` (q4web.ts:58-66): [nibbles | scales | mins]."""
    return np.concatenate([_c(nib, np.uint8), _c(sc, "<u2").view(np.uint8), _c(mn, "<u2").view(np.uint8)])


def pack_q3(lo, hi, sc, mn) -> np.ndarray:
    """``packQ3`` (q3web.ts:65-76): [lo | hi | scales | mins]."""
    return np.concatenate([_c(lo, "<u4").view(np.uint8), _c(hi, "<u4").view(np.uint8),
                           _c(sc, "<u2").view(np.uint8), _c(mn, "<u2").view(np.uint8)])


def unpack_q8(blob, n):
    """``unpackQ8`` (q8web.ts:65-72)."""
    b = _c(blob, np.uint8)
    g = n // GROUP
    return b[:n].view(np.int8).copy(), b[n:n + 2 * g].view("<u2").copy()


def unpack_q4(blob, n):
    """``unpackQ4`` (q4web.ts:70-80): scales at n/2, mins at n/2 + 2*groups."""
    b = _c(blob, np.uint8)
    g = n // GROUP
    nl = n // 2
    return b[:nl].copy(), b[nl:nl + 2 * g].copy().view("<u2"), b[nl + 2 * g:nl + 4 * g].copy().view("<u2")


def unpack_q3(blob, n):
    """``unpackQ3`` (q3web.ts:80-95): lo words, hi words, scales, mins."""
    b = _c(blob, np.uint8)
    g = n // GROUP
    lb, hb = (n // 16) * 4, (n // 32) * 4
    lo = b[:lb].copy().view("<u4")
    hi = b[lb:lb + hb].copy().view("<u4")
    sc = b[lb + hb:lb + hb + 2 * g].copy().view("<u2")
    mn = b[lb + hb + 2 * g:lb + hb + 4 * g].copy().view("<u2")
    return lo, hi, sc, mn


# ---- sampling pre-work (decodeTopKQ8's passes) ---------------------------------------------------

def softcap_logits(logits: np.ndarray, cap: float) -> np.ndarray:
    """``cap * Math.tanh(l / cap)`` in double, stored to a Float32Array: the CPU reference of the
    reference's own top-k validation (``kernels.ts:2833-2834``; GPU pass ``shaders.ts:954-964``)."""
    v = np.asarray(logits, np.float32).astype(np.float64)
    return (cap * np.tanh(v / cap)).astype(np.float32)


def penalize_logits(logits: np.ndarray, recent, penalty: float) -> np.ndarray:
    """Repetition penalty as ``sampleNextToken`` applies it (``sampling.ts:84-90``): each id once,
    ids outside ``[0, n)`` skipped, ``l > 0 ? l / p : l * p`` in double, stored to float32."""
    out = np.asarray(logits, np.float32).copy()
    n = out.size
    for i in dict.fromkeys(int(r) for r in recent):
        if 0 <= i < n:
            v = float(out[i])
            out[i] = np.float32(v / penalty if v > 0 else v * penalty)
    return out


def top_k(logits: np.ndarray, k: int):
    """The k largest values and their ids, sorted descending, ties by smaller id: the stable sort of
    the reference's validation (``kernels.ts:2836``, ``Array.sort`` is stable). NaN ranks last."""
    v = np.asarray(logits, np.float32)
    key = np.where(np.isnan(v), -np.inf, v.astype(np.float64))
    nan_last = np.isnan(v).astype(np.int8)
    order = np.lexsort((np.arange(v.size), -key, nan_last))[:k]
    return order.astype(np.uint32), v[order]


# ---- the elementwise ops around recMM in a decoder layer (fused into GEMV plans) -------------------

def rmsnorm(x: np.ndarray, w: np.ndarray, rows: int, dim: int, eps: float = 1e-5, one_plus: bool = False):
    """``rmsnormCpu`` (``kernels.ts:3395-3404``): sum of squares in double, ``1 / sqrt(ss / dim + eps)``,
    ``x * inv * g`` with ``g = w`` or ``1 + w``, stored to float32."""
    x = np.asarray(x, np.float32).astype(np.float64).reshape(rows, dim)
    g = np.asarray(w, np.float32).astype(np.float64)
    g = 1.0 + g if one_plus else g
    out = np.empty_like(x)
    for r in range(rows):
        ss = 0.0
        for v in x[r]:
            ss += v * v
        inv = 1.0 / np.sqrt(ss / dim + eps)
        out[r] = x[r] * inv * g
    return out.astype(np.float32).ravel()


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``(g / (1 + Math.exp(-g))) * up`` in double, stored to float32 (``kernels.ts:3526-3528``)."""
    g = np.asarray(gate, np.float32).astype(np.float64)
    return ((g / (1.0 + np.exp(-g))) * np.asarray(up, np.float32)).astype(np.float32)


def geglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``geluTanh(g) * up`` (``kernels.ts:3498-3500, 3526``), double, stored to float32."""
    g = np.asarray(gate, np.float32).astype(np.float64)
    gelu = 0.5 * g * (1.0 + np.tanh(0.7978845608 * (g + 0.044715 * g * g * g)))
    return (gelu * np.asarray(up, np.float32)).astype(np.float32)


# ---- convolution (fused-dequant consumers) ------------------------------------------------------

def conv2d(inp, w, bias, Cin, H, W, Cout, kh, kw, stride=1, pad=0, return_absden=False):
    """The reference conv of the self-validation (kernels.ts:3049-3061): ``out[Cout, OH, OW]`` with
    the f64 sum over (ci, ky, kx) starting from ``bias[co]``, stored to f32; ``w`` is the
    dequantized flat OIHW weight (float32). With ``return_absden``, also sum |inp * w| + |bias|."""
    OH, OW = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
    inp = _c(inp, np.float32).ravel()
    w = _c(w, np.float32).ravel()
    assert inp.size == Cin * H * W and w.size == Cout * Cin * kh * kw
    b = None if bias is None else _c(bias, np.float32).ravel()
    out = np.empty(Cout * OH * OW, np.float32)
    den = np.empty(Cout * OH * OW, np.float64) if return_absden else None
    _L().oracle_conv2d(_p(inp), _p(w), _p(b), Cin, H, W, Cout, kh, kw, stride, pad, _p(out), _p(den))
    out = out.reshape(Cout, OH, OW)
    return (out, den.reshape(Cout, OH, OW)) if return_absden else out


def matmul_t_f16w(x, w_bits, M, K, N):
    """MATMUL_T_F16W (shaders.ts:2240-2259): y = x . W^T with W [N, K] IEEE f16 bits widened to f32
    (exact), the sum in f64 here. Returns (y float64 [M, N], sum |x w| [M, N])."""
    x = np.asarray(x, np.float32).reshape(M, K).astype(np.float64)
    w = np.asarray(w_bits, np.uint16).reshape(N, K).view(np.float16).astype(np.float64)
    return x @ w.T, np.abs(x) @ np.abs(w).T
