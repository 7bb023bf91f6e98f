"""Pins the oracle's f16 decode / encode (restating src/lib/brik/f16.ts) without importing the reference.

* decode: exhaustive over all 65,536 bit patterns against IEEE binary16 (numpy), the textbook
  routine the reference's formula implements. A wrong bias, mantissa divisor or sign fails.
* encode: the reference's own known-answer checks (codec.test.ts:30-36), IEEE agreement away from
  ties, and the half-up tie / flush / clamp rules written as closed forms on the bit pattern.
"""
import numpy as np

from oracle import f16_to_f64, f32_to_f16
from brimkern_amd.synth import f16_bits


def test_decode_exhaustive_against_ieee():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = f16_to_f64(h)
    ieee = h.view(np.float16).astype(np.float64)
    e = (h >> 10) & 0x1F
    normal = (e > 0) & (e < 31)
    assert np.array_equal(got[normal], ieee[normal])
    sub = e == 0
    # subnormals use the literal 5.9604645e-8 for 2^-24 (f16.ts:30): within 1e-8 relative, and the
    # same float32 once rounded
    assert np.allclose(got[sub], ieee[sub], rtol=1e-8, atol=0)
    assert np.array_equal(got[sub].astype(np.float32), ieee[sub].astype(np.float32))
    inf = (e == 31) & ((h & 0x3FF) == 0)
    nan = (e == 31) & ((h & 0x3FF) != 0)
    assert np.array_equal(got[inf], ieee[inf]) and np.all(np.isinf(got[inf]))
    assert np.all(np.isnan(got[nan]))


def test_encode_known_bits():
    # src/lib/brik/codec.test.ts:30-36
    assert f32_to_f16([1.0])[0] == 0x3C00
    assert f32_to_f16([-2.0])[0] == 0xC000
    assert f32_to_f16([0.0])[0] == 0
    assert f16_to_f64(f32_to_f16([0.5]))[0] == 0.5
    assert f32_to_f16([65504.0])[0] == 0x7BFF
    assert f32_to_f16([1e6])[0] == 0x7BFF          # clamp, not Inf (f16.ts:17)
    assert f32_to_f16([-1e6])[0] == 0xFBFF
    assert f32_to_f16([2.0 ** -15])[0] == 0         # below 2^-14 flushes (f16.ts:16)
    assert f32_to_f16([2.0 ** -14])[0] == 0x0400


def _rand_f32_in(lo, hi, n, seed):
    rng = np.random.default_rng(seed)
    return rng.uniform(lo, hi, n).astype(np.float32)


def test_encode_matches_ieee_away_from_ties():
    v = np.concatenate([_rand_f32_in(2.0 ** -14, 60000.0, 200000, 1), -_rand_f32_in(2.0 ** -14, 1.0, 200000, 2)])
    bits = v.view(np.uint32)
    tie = (bits & 0x1FFF) == 0x1000
    got = f32_to_f16(v)
    ieee = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got[~tie], ieee[~tie])


def test_encode_ties_round_half_up():
    # exact ties: dropped 13 bits == 0x1000. The reference adds the top dropped bit (f16.ts:18),
    # i.e. rounds half up in magnitude; IEEE would round to even.
    rng = np.random.default_rng(3)
    top = rng.integers(0, 1 << 10, 5000, dtype=np.uint32)      # kept mantissa bits
    exp = rng.integers(127 - 14, 127 + 15, 5000, dtype=np.uint32)
    bits = (exp << 23) | (top << 13) | 0x1000
    v = bits.view(np.float32)
    got = f32_to_f16(v).astype(np.uint32)
    mant = top + 1
    e16 = exp - 127 + 15 + (mant >> 10)
    want = (e16 << 10) | (mant & 0x3FF)
    assert np.array_equal(got, want)


def test_synth_encoder_equals_oracle_encoder():
    v = np.concatenate([_rand_f32_in(-2.0, 2.0, 100000, 4), _rand_f32_in(0.005, 0.04, 100000, 5),
                        np.array([0.0, -0.0, 1e-9, -1e-9, 1e6, -1e6, 65504.0, 65520.0], np.float32)])
    bits = v.view(np.uint32)
    ties = ((np.arange(2000, dtype=np.uint32) << 13) | 0x1000 | (np.uint32(120) << 23)).view(np.float32)
    v = np.concatenate([v, ties])
    assert np.array_equal(f16_bits(v), f32_to_f16(v))
    del bits
