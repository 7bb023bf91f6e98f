"""Pins of the oracle's sampling pre-work (softcap, repetition penalty, top-k; decodeTopKQ8's passes).

Each function is fixed by checks that do not restate its formula:
- ``top_k``: brute force over every permutation rank (Python ``sorted`` on (-value, id)), on inputs
  full of ties, infinities and NaN; invariants (descending, distinct ids, values at those ids);
- ``softcap_logits``: tanh's closed-form properties: odd, bounded by the cap, slope 1 at 0, the
  identity cap * tanh(v / cap) = cap * (e^(2v/cap) - 1) / (e^(2v/cap) + 1), monotone;
- ``penalize_logits``: the reference's rule on signs (a positive logit shrinks toward 0, a negative
  one grows away from 0, zero stays), the involution with 1/p, each id applied once, out-of-range ids
  ignored (``sampling.ts:84-90``).
"""
import math

import numpy as np
import pytest

from oracle import brik_oracle as O


def brute_top_k(v, k):
    key = [(1 if math.isnan(x) else 0, -(x if not math.isnan(x) else 0.0), i) for i, x in enumerate(v.tolist())]
    order = [i for _, _, i in sorted(key)][:k]
    return np.array(order, np.uint32)


@pytest.mark.parametrize("seed", range(6))
def test_top_k_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 300))
    v = rng.integers(-5, 5, size=n).astype(np.float32)        # many ties
    v[rng.random(n) < 0.05] = np.nan
    v[rng.random(n) < 0.03] = np.inf
    v[rng.random(n) < 0.03] = -np.inf
    k = int(rng.integers(1, min(64, n) + 1))
    ids, vals = O.top_k(v, k)
    assert np.array_equal(ids, brute_top_k(v, k))
    assert np.array_equal(vals, v[ids], equal_nan=True)
    assert len(set(ids.tolist())) == k


def test_top_k_sorted_and_maximal():
    rng = np.random.default_rng(7)
    v = rng.standard_normal(5000).astype(np.float32)
    ids, vals = O.top_k(v, 64)
    assert np.all(np.diff(vals) <= 0)
    assert vals[-1] >= np.sort(v)[-64]
    rest = np.setdiff1d(np.arange(v.size), ids)
    assert v[rest].max() <= vals[-1]


def test_softcap_properties():
    cap = 30.0
    v = np.linspace(-400, 400, 4001, dtype=np.float32)
    s = O.softcap_logits(v, cap)
    assert np.all(np.abs(s) <= cap)
    assert np.array_equal(s, -O.softcap_logits(-v, cap))                      # odd
    assert np.all(np.diff(s.astype(np.float64)) >= 0)                         # monotone
    small = np.float32(1e-3)
    assert abs(float(O.softcap_logits(np.array([small]), cap)[0]) - float(small)) < 1e-9   # slope 1 at 0
    x = v.astype(np.float64) / cap
    ident = cap * np.expm1(2 * x) / (np.exp(2 * x) + 1)
    ok = np.abs(x) < 20
    np.testing.assert_allclose(s[ok], ident[ok].astype(np.float32), rtol=2e-7, atol=1e-6)


def test_penalty_rule():
    v = np.array([2.0, -2.0, 0.0, 5.0, 7.0], np.float32)
    p = 1.25
    out = O.penalize_logits(v, [0, 1, 2, 0, 99, -1], p)     # 0 repeated, 99 and -1 out of range
    assert 0 < out[0] < v[0]                                 # positive shrinks
    assert out[1] < v[1] < 0                                 # negative grows away from 0
    assert out[2] == 0.0
    assert out[3] == v[3] and out[4] == v[4]                 # untouched
    back = O.penalize_logits(out, [0, 1], 1.0 / p)
    np.testing.assert_allclose(back[:2], v[:2], rtol=1e-6)   # involution with 1 / p
    once = O.penalize_logits(v, [0], p)
    assert once[0] == out[0]                                  # a repeated id is applied once
