"""Pins the oracle's plane layouts and dequantization (q8web.ts / q4web.ts / q3web.ts).

Two kinds of check, neither a retyping of the oracle:
* the reference's own codec unit tests re-derived (src/lib/brik/q4web.test.ts, q8web.test.ts,
  q3web.test.ts): round-trip error bounds, exact evenly spaced levels, plane sizes, bits/weight,
  pack -> unpack byte-exactness, the row sub-blob reconstruction of model.ts:427-448;
* closed forms: integer codes drawn first, packed by an independent numpy packer
  (brimkern_amd.layout / synth), then dequantized by the C oracle and compared with q*s+m computed
  directly from the codes. A wrong nibble order, bit position, group index or sign extension fails.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import layout, synth

N01 = synth.normal(11, 8192)


def _err(a, b):
    d = np.abs(a.astype(np.float64) - b.astype(np.float64))
    return d.mean(), d.max()


# ---- re-derived reference codec tests --------------------------------------------------

def test_q4_roundtrip_error():          # q4web.test.ts:23-33
    back = O.dequant_q4(*O.quantize_q4(N01))
    mean, mx = _err(back, N01)
    assert mean < 0.08 and mx < 0.35


def test_q4_sixteen_levels_exact():     # q4web.test.ts:35-43
    data = (np.arange(32) % 16 / 15).astype(np.float32)
    back = O.dequant_q4(*O.quantize_q4(data))
    assert np.abs(back - data).max() < 1e-2


def test_q4_plane_sizes():              # q4web.test.ts:45-59
    nib, sc, mn = O.quantize_q4(np.zeros(32, np.float32))
    assert nib.size == 16 and sc.size == 1 and mn.size == 1
    bpw = O.q4_byte_length(4096) * 8 / 4096
    assert 4 < bpw < 6 and O.q4_byte_length(4096) < 4096 * 2


def test_q8_roundtrip_error():          # q8web.test.ts:23-41
    back = O.dequant_q8(*O.quantize_q8(N01))
    mean, mx = _err(back, N01)
    assert mean < 0.015 and mx < 0.05
    d2 = synth.normal(12, 4096)
    assert _err(O.dequant_q8(*O.quantize_q8(d2)), d2)[0] < 0.02


def test_q8_plane_sizes():              # q8web.test.ts:43-57
    codes, sc = O.quantize_q8(np.zeros(32, np.float32))
    assert codes.size == 32 and sc.size == 1
    bpw = O.q8_byte_length(4096) * 8 / 4096
    assert 8 < bpw < 9


def test_q8_row_subblob():              # q8web.test.ts:59-80, model.ts:427-435
    rows, d = 4, 64
    n = rows * d
    data = synth.normal(13, n)
    full = O.pack_q8(*O.quantize_q8(data))
    deq_full = O.dequant_q8(*O.unpack_q8(full, n))
    g = d // 32
    for r in range(rows):
        blob = np.concatenate([full[r * d:(r + 1) * d], full[n + r * g * 2:n + (r + 1) * g * 2]])
        assert np.array_equal(O.dequant_q8(*O.unpack_q8(blob, d)), deq_full[r * d:(r + 1) * d])


def test_q3_roundtrip_error():          # q3web.test.ts:23-33
    back = O.dequant_q3(*O.quantize_q3(N01))
    mean, mx = _err(back, N01)
    assert mean < 0.22 and mx < 0.8


def test_q3_eight_levels_exact():       # q3web.test.ts:35-43
    data = (np.arange(32) % 8 / 7).astype(np.float32)
    back = O.dequant_q3(*O.quantize_q3(data))
    assert np.abs(back - data).max() < 1e-2


def test_q3_plane_sizes_and_pack_roundtrip():   # q3web.test.ts:45-68
    lo, hi, sc, mn = O.quantize_q3(np.zeros(96, np.float32))
    assert lo.size == 6 and hi.size == 3 and sc.size == 3 and mn.size == 3
    t = O.quantize_q3(synth.normal(14, 4096))
    u = O.unpack_q3(O.pack_q3(*t), 4096)
    for a, b in zip(t, u):
        assert np.array_equal(a, b)
    assert O.q3_byte_length(4096) == 4096 // 2


def test_q4_q8_pack_roundtrip():
    t4 = O.quantize_q4(N01)
    for a, b in zip(t4, O.unpack_q4(O.pack_q4(*t4), N01.size)):
        assert np.array_equal(a, b)
    t8 = O.quantize_q8(N01)
    for a, b in zip(t8, O.unpack_q8(O.pack_q8(*t8), N01.size)):
        assert np.array_equal(a, b)


# ---- independent layout implementation agrees ------------------------------------------

@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_layout_module_matches_oracle_offsets(fmt):
    n = 32 * 37
    assert layout.byte_length(fmt, n) == {"q8": O.q8_byte_length, "q4": O.q4_byte_length,
                                          "q3": O.q3_byte_length}[fmt](n)
    t = synth.tensor(fmt, 5, 37, 32)
    blob = layout.pack(fmt, t)
    planes = layout.split_blob(fmt, blob, n)
    ref = {"q8": O.unpack_q8, "q4": O.unpack_q4, "q3": O.unpack_q3}[fmt](blob, n)
    for a, b in zip(planes.values(), ref):
        assert np.array_equal(np.asarray(a), np.asarray(b))


# ---- closed forms on known integer codes --------------------------------------------------

def _sm(sc, mn, n):
    s = sc.view(np.float16).astype(np.float64)
    m = mn.view(np.float16).astype(np.float64) if mn is not None else np.zeros_like(s)
    return np.repeat(s, 32)[:n], np.repeat(m, 32)[:n]


def test_q4_dequant_closed_form():
    n = 32 * 64
    rng = np.random.default_rng(21)
    q = rng.integers(0, 16, n)
    nib = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)          # low nibble = even index
    sc = synth.scales(22, n // 32, 0.005, 0.02)
    mn = synth.f16_bits(rng.uniform(-0.2, 0.2, n // 32).astype(np.float32))
    s, m = _sm(sc, mn, n)
    want = (q * s + m).astype(np.float32)                     # exact in f64, one rounding
    assert np.array_equal(O.dequant_q4(nib, sc, mn), want)


def test_q8_dequant_closed_form():
    n = 32 * 64
    rng = np.random.default_rng(23)
    q = rng.integers(-128, 128, n)                              # includes -128 (sign extension)
    sc = synth.scales(24, n // 32, 0.005, 0.02)
    s, _ = _sm(sc, None, n)
    assert np.array_equal(O.dequant_q8(q.astype(np.int8), sc), (q * s).astype(np.float32))


def test_q3_dequant_closed_form():
    n = 32 * 64
    rng = np.random.default_rng(25)
    q = rng.integers(0, 8, n).astype(np.uint64)
    idx = np.arange(n, dtype=np.uint64)
    lo = np.zeros(n // 16, np.uint64)
    hi = np.zeros(n // 32, np.uint64)
    for i in range(n):  # plain loop: an independent packer for the bit planes
        lo[i >> 4] |= (int(q[i]) & 3) << ((i & 15) * 2)
        hi[i >> 5] |= (int(q[i]) >> 2) << (i & 31)
    sc = synth.scales(26, n // 32, 0.01, 0.04)
    mn = synth.centred_mins(sc, 3.5)
    s, m = _sm(sc, mn, n)
    want = (q.astype(np.float64) * s + m).astype(np.float32)
    got = O.dequant_q3(lo.astype(np.uint32), hi.astype(np.uint32), sc, mn)
    assert np.array_equal(got, want)
    del idx


def test_known_answers():
    sc = synth.f16_bits(np.array([0.01], np.float32))
    mn = synth.f16_bits(np.array([-0.05], np.float32))
    s = float(sc.view(np.float16)[0]); m = float(mn.view(np.float16)[0])
    assert np.all(O.dequant_q4(np.zeros(16, np.uint8), sc, mn) == np.float32(m))          # codes 0 -> m
    assert np.all(O.dequant_q4(np.full(16, 0xFF, np.uint8), sc, mn) == np.float32(15 * s + m))
    lo, hi = np.full(2, 0xFFFFFFFF, np.uint32), np.full(1, 0xFFFFFFFF, np.uint32)
    assert np.all(O.dequant_q3(lo, hi, sc, mn) == np.float32(7 * s + m))
    c = np.full(32, -128, np.int8)
    assert np.all(O.dequant_q8(c, sc) == np.float32(-128 * s))
    c[:] = 127
    assert np.all(O.dequant_q8(c, sc) == np.float32(127 * s))
