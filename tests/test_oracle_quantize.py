"""Pins of the oracle's encoder (quantizeQ8 / quantizeQ4 / quantizeQ3, q8web.ts:28-50, q4web.ts:28-53,
q3web.ts:34-60), the checker of the GPU quantizers.

The reference holds no encoder vectors (its tests draw from unseeded Math.random), so the oracle is
pinned by checks that do not restate its formula:
  * ties: codes of values placed exactly halfway between two levels, worked out by hand for
    Math.round (ties toward +infinity); round-half-even or half-away-from-zero fail these;
  * brute force: every code is the level nearest to the value in exact rational arithmetic, the
    larger level on a tie, for the scale and min the encoder chose;
  * the scale and min are the f16 values nearest (within half an f16 step) to the group's
    (max - min) / L (or amax / 127) and min;
  * special groups (all-zero, constant, NaN, infinities) worked out by hand from the reference text;
  * a second restatement in the reference's own language (oracle/cpuref.js: JS doubles, the real
    Math.round and typed-array stores) produces the same bytes.
"""
import os
import shutil
import subprocess
import tempfile
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LEVELS = {"q8": 127, "q4": 15, "q3": 7}


def codes_of(fmt, x):
    """(codes int array, scales u16, mins u16 or None) from the oracle's encoder."""
    if fmt == "q8":
        c, s = O.quantize_q8(x)
        return c.astype(np.int64), s, None
    if fmt == "q4":
        nib, s, m = O.quantize_q4(x)
        c = np.empty(nib.size * 2, np.int64)
        c[0::2], c[1::2] = nib & 15, nib >> 4
        return c, s, m
    lo, hi, s, m = O.quantize_q3(x)
    idx = np.arange(x.size)
    c = ((lo[idx >> 4] >> ((idx & 15) * 2)) & 3) | (((hi[idx >> 5] >> (idx & 31)) & 1) << 2)
    return c.astype(np.int64), s, m


def test_ties_round_toward_plus_infinity_q8():
    # s = 0.0625 exactly: amax = 127 s, and amax / 127 is an f16 value
    s = 0.0625
    k = np.array([-6, -3, -2, -1, 0, 1, 2, 5], np.float64)
    x = np.zeros(32, np.float32)
    x[0] = 127 * s
    x[1:9] = (k + 0.5) * s                  # exactly halfway between levels k and k + 1
    x[9:17] = -(k + 0.5) * s
    c, sc, _ = codes_of("q8", x)
    assert O.f16_to_f64(sc)[0] == s
    assert c[0] == 127
    assert c[1:9].tolist() == [-5, -2, -1, 0, 1, 2, 3, 6]          # k + 1 for every k
    assert c[9:17].tolist() == [6, 3, 2, 1, 0, -1, -2, -5]         # -(k + 0.5) -> -k


@pytest.mark.parametrize("fmt", ["q4", "q3"])
def test_ties_round_toward_plus_infinity_asym(fmt):
    L = LEVELS[fmt]
    m, s = -1.0, 0.125                       # both f16 values; max = m + L s makes (max - min) / L == s
    x = np.full(32, m, np.float32)
    x[1] = m + L * s
    x[2:2 + L - 1] = m + (np.arange(L - 1) + 0.5) * s      # halfway between k and k + 1, k = 0 .. L-2
    c, sc, mn = codes_of(fmt, x)
    assert O.f16_to_f64(sc)[0] == s and O.f16_to_f64(mn)[0] == m
    assert c[0] == 0 and c[1] == L
    assert c[2:2 + L - 1].tolist() == list(range(1, L))


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_codes_are_the_nearest_levels(fmt):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(32 * 40) * rng.choice([0.01, 1, 300], 32 * 40)).astype(np.float32)
    x[::97] *= 50                            # a few far values: clamped codes at the ends
    c, sc, mn = codes_of(fmt, x)
    L = LEVELS[fmt]
    lo = -127 if fmt == "q8" else 0
    for g in range(x.size // 32):
        s = Fraction(O.f16_to_f64(sc[g:g + 1])[0])
        m = Fraction(O.f16_to_f64(mn[g:g + 1])[0]) if mn is not None else Fraction(0)
        for i in range(32):
            v = Fraction(float(x[32 * g + i]))
            # nearest level in exact arithmetic, the larger one on a tie
            best = max(range(lo, L + 1), key=lambda q: (-abs(q * s + m - v), q))
            assert c[32 * g + i] == best, (fmt, g, i)


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_scale_and_min_are_nearest_f16(fmt):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(32 * 200) * 2).astype(np.float32).reshape(-1, 32)
    _, sc, mn = codes_of(fmt, x.ravel())
    d = x.astype(np.float64)
    want = np.abs(d).max(1) / 127 if fmt == "q8" else (d.max(1) - d.min(1)) / LEVELS[fmt]
    got = O.f16_to_f64(sc)
    half_step = np.exp2(np.floor(np.log2(want)) - 11)             # half an f16 step at that magnitude
    assert np.all(np.abs(got - want) <= half_step * (1 + 1e-6))
    if mn is not None:
        mins = d.min(1)
        assert np.all(np.abs(O.f16_to_f64(mn) - mins) <= np.exp2(np.floor(np.log2(np.abs(mins))) - 11) * (1 + 1e-6))


def test_signed_zero_minimum_is_the_first():
    # the reference scans left to right with `v < mn`: of +0 and -0, whichever comes first stays
    x = np.zeros(64, np.float32)
    x[0], x[1], x[2] = -0.0, 0.0, 1.0
    x[32], x[33], x[34] = 0.0, -0.0, 1.0
    for fmt in ("q4", "q3"):
        _, _, mn = codes_of(fmt, x)
        assert mn.tolist() == [0x8000, 0x0000], fmt


def test_special_groups():
    x = np.zeros(32 * 6, np.float32)
    x[32:64] = 2.5                               # constant
    x[64:96] = np.nan                            # all NaN
    x[96:128] = np.linspace(-1, 1, 32)
    x[100] = np.nan                              # one NaN: skipped by the min / max loop
    x[128:160] = 1.0
    x[130] = np.inf                              # an infinity
    x[160:192] = -np.inf
    c8, s8, _ = codes_of("q8", x)
    c4, s4, m4 = codes_of("q4", x)
    # all zero: scale 0 || 1e-8 = 1e-8 encodes to +0; codes 0
    assert s8[0] == 0 and s4[0] == 0 and m4[0] == 0 and not c8[:32].any() and not c4[:32].any()
    # constant 2.5: q4 scale 1e-8 -> 0, min f16(2.5) = 0x4100, codes 0; q8 scale f16(2.5 / 127), codes 127
    assert s4[1] == 0 and m4[1] == 0x4100 and not c4[32:64].any()
    assert (c8[32:64] == 127).all()
    # all NaN: q8 amax stays 0 -> scale bits 0, codes 0; q4 min = Infinity, max = -Infinity ->
    # scale -Infinity -> 0xfbff, min Infinity -> 0x7bff, codes 0
    assert s8[2] == 0 and not c8[64:96].any()
    assert s4[2] == 0xFBFF and m4[2] == 0x7BFF and not c4[64:96].any()
    # one NaN: the same scale and min as without it, and code 0 in its place
    y = x[96:128].copy()
    y[4] = y[5]
    cy, sy, my = codes_of("q4", y)
    assert s4[3] == sy[0] and m4[3] == my[0] and c4[100] == 0
    assert np.array_equal(np.delete(c4[96:128], 4), np.delete(cy, 4))
    # +inf: q8 scale clamps to 65504 (0x7bff); the inf codes 127, the 1.0s round(1 / 65504) = 0
    assert s8[4] == 0x7BFF and c8[130] == 127 and not np.delete(c8[128:160], 2).any()
    # all -inf: q4 min = max = -inf -> (max - min) = NaN -> 1e-8 -> +0; min 0xfbff; codes 0
    assert s4[5] == 0 and m4[5] == 0xFBFF and not c4[160:192].any()


@pytest.mark.skipif(shutil.which("node") is None, reason="node not installed")
@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_numpy_and_js_restatements_agree(fmt):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(32 * 3000) * 3).astype(np.float32)
    x[5] = np.nan
    x[100:132] = np.nan
    x[200], x[300] = np.inf, -np.inf
    x[400:432] = 0
    x[500:532] = 2.5
    x[640:672] = np.round(x[640:672] * 8) / 8                     # many exact ties
    x[700:732] = 1e-30                                            # scale below the f16 range
    x[800:832] = 3e38                                             # (max - min) overflows nothing, scale clamps
    x[832:864] = 0
    x[832], x[850] = -0.0, -0.0                                   # signed zeros: the first minimum's sign
    x[864:896] = np.abs(x[864:896])
    x[870], x[871] = 0.0, -0.0
    py = {"q8": lambda: O.pack_q8(*O.quantize_q8(x)), "q4": lambda: O.pack_q4(*O.quantize_q4(x)),
          "q3": lambda: O.pack_q3(*O.quantize_q3(x))}[fmt]()
    with tempfile.TemporaryDirectory() as d:
        inp, out = os.path.join(d, "x.f32"), os.path.join(d, "q.bin")
        x.tofile(inp)
        subprocess.check_call(["node", os.path.join(ROOT, "oracle", "cpuref.js"), "quantize", fmt, inp, out],
                              stdout=subprocess.DEVNULL)
        js = np.fromfile(out, np.uint8)
    assert np.array_equal(js, py)
