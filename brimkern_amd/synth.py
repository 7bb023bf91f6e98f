"""Seeded synthetic inputs in the exact ``.brik`` plane layouts.

The reference draws every test input from unseeded ``Math.random`` (e.g.
``src/lib/brik/q4web.test.ts:14-21``), so there is no reference stream to reproduce. This module
fixes one: SplitMix64 as a counter-based generator (value i of stream ``seed`` is
``mix64(seed + (i + 1) * 0x9E3779B97F4A7C15)``), uniforms from the top 53 bits, normals by
Box-Muller in float64 rounded once to float32.

Codes are drawn uniformly as the benchmark configurations specify, so the planes are built
directly from random bits (uniform q4 codes are uniform nibble bytes; uniform q3 codes are
uniform lo/hi plane bits). Scales are ``f16(U(a, b))`` and mins ``f16(-c * s)`` (the configs do
not fix mins; centring them keeps the dequantized weights zero-mean).
"""
from __future__ import annotations

import numpy as np

GROUP = 32
_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Values ``offset .. offset+n-1`` of the SplitMix64 stream for ``seed`` (uint64)."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0, offset: int = 0) -> np.ndarray:
    """float64 uniforms in [lo, hi)."""
    u = (splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return lo + (hi - lo) * u


def normal(seed: int, n: int) -> np.ndarray:
    """float32 N(0,1) by Box-Muller (float64 math, one rounding)."""
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    u1 = 1.0 - u[0::2]          # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(2 * np.pi * u2)
    z[1::2] = r * np.sin(2 * np.pi * u2)
    return z[:n].astype(np.float32)


def random_bytes(seed: int, nbytes: int) -> np.ndarray:
    words = splitmix64(seed, (nbytes + 7) // 8)
    return words.view(np.uint8)[:nbytes].copy()


def f16_bits(v: np.ndarray) -> np.ndarray:
    """f32 -> f16 bits with the reference encoder's rules (``f32ToF16Bits``,
    src/lib/brik/f16.ts:8-22): the 13 dropped mantissa bits round half-up, |x| < 2^-14 flushes to
    +-0, exponents past the f16 range clamp to +-0x7bff. (This differs from IEEE round-to-nearest-
    even only on exact ties and subnormals.)"""
    x = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.int64)
    sign = (x >> 16) & 0x8000
    exp = ((x >> 23) & 0xFF) - 127 + 15
    mant = x & 0x7FFFFF
    r = (mant >> 13) + ((mant >> 12) & 1)
    carry = r == 0x400
    r = np.where(carry, 0, r)
    e2 = exp + carry
    out = sign | (e2 << 10) | (r & 0x3FF)
    out = np.where(exp >= 31, sign | 0x7BFF, out)
    out = np.where(exp <= 0, sign, out)
    return out.astype(np.uint16)


def scales(seed: int, groups: int, lo: float, hi: float) -> np.ndarray:
    return f16_bits(uniform(seed, groups, lo, hi).astype(np.float32))


def centred_mins(sc_bits: np.ndarray, centre: float) -> np.ndarray:
    s = sc_bits.view(np.float16).astype(np.float32)
    return f16_bits(-centre * s)


def q8_tensor(seed: int, N: int, K: int, s_lo=0.005, s_hi=0.02):
    """codes uniform in [-127, 127], group-32 scales f16(U(s_lo, s_hi)). Returns dict of planes."""
    n = N * K
    w = splitmix64(seed, n)
    codes = ((w >> np.uint64(32)) % np.uint64(255)).astype(np.int16) - 127
    g = n // GROUP
    return {"fmt": "q8", "N": N, "K": K, "codes": codes.astype(np.int8),
            "sc": scales(seed ^ 0x5C, g, s_lo, s_hi)}


def q4_tensor(seed: int, N: int, K: int, s_lo=0.005, s_hi=0.02, centre=7.5):
    n = N * K
    g = n // GROUP
    sc = scales(seed ^ 0x5C, g, s_lo, s_hi)
    return {"fmt": "q4", "N": N, "K": K, "nib": random_bytes(seed, n // 2),
            "sc": sc, "mn": centred_mins(sc, centre)}


def q3_tensor(seed: int, N: int, K: int, s_lo=0.01, s_hi=0.04, centre=3.5):
    n = N * K
    g = n // GROUP
    sc = scales(seed ^ 0x5C, g, s_lo, s_hi)
    lo = random_bytes(seed, (n // 16) * 4).view("<u4")
    hi = random_bytes(seed ^ 0x41, (n // 32) * 4).view("<u4")
    return {"fmt": "q3", "N": N, "K": K, "lo": lo, "hi": hi, "sc": sc, "mn": centred_mins(sc, centre)}


def tensor(fmt: str, seed: int, N: int, K: int, **kw):
    return {"q8": q8_tensor, "q4": q4_tensor, "q3": q3_tensor}[fmt](seed, N, K, **kw)


def moe_routing(seed: int, tokens: int, experts: int, topk: int):
    """Top-k routing from a softmax over N(0,1) gate logits [tokens, experts].

    Returns (row_token int32[tokens*topk] sorted by expert, row_off int32[experts+1]). Rows of
    expert e are row_token[row_off[e]:row_off[e+1]], tokens ascending within an expert."""
    logits = normal(seed, tokens * experts).reshape(tokens, experts).astype(np.float64)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    # top-k by probability; ties broken by lower expert index (stable sort on -p)
    top = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    tok = np.repeat(np.arange(tokens, dtype=np.int64), topk)
    exp = top.ravel()
    order = np.lexsort((tok, exp))
    counts = np.bincount(exp, minlength=experts)
    row_off = np.zeros(experts + 1, np.int32)
    row_off[1:] = np.cumsum(counts)
    return tok[order].astype(np.int32), row_off
