"""The committed golden fixtures reproduce bit-exactly through the CPU oracle (regression guard),
and the fixture blobs split with the product's layout module exactly as the oracle's unpack does."""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import layout
from helpers import load_golden, PLANES

CASES, MOE = load_golden()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_case(case):
    fmt, M, K, N = case["fmt"], case["M"], case["K"], case["N"]
    planes = layout.split_blob(fmt, case["blob"], N * K)
    unpack = {"q8": O.unpack_q8, "q4": O.unpack_q4, "q3": O.unpack_q3}[fmt](case["blob"], N * K)
    for k, ref in zip(PLANES[fmt], unpack):
        assert np.array_equal(np.asarray(planes[k]), np.asarray(ref))
    args = [planes[k] for k in PLANES[fmt]]
    deq = {"q8": O.dequant_q8, "q4": O.dequant_q4, "q3": O.dequant_q3}[fmt](*args)
    assert np.array_equal(deq, case["deq"])
    y = {"q8": O.matmul_t_q8, "q4": O.matmul_t_q4, "q3": O.matmul_t_q3}[fmt](case["x"], *args, M, K, N)
    assert np.array_equal(y.ravel(), case["y"])


def test_golden_moe():
    m = MOE
    p = layout.split_blob("q4", m["blob"], m["E"] * m["N"] * m["K"])
    y = O.moe_matmul_t_q4(m["x"], m["row_off"], p["nib"], p["sc"], p["mn"], m["E"], m["K"], m["N"])
    assert np.array_equal(y.ravel(), m["y"])
