"""The JavaScript restatement of the reference CPU matmul (oracle/cpuref.js, the CPU baseline bench.py
times) reproduces the golden fixtures bit-exactly: the same f64 left-to-right sums as the C oracle."""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

from helpers import load_golden

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CASES, _ = load_golden()
pytestmark = pytest.mark.skipif(shutil.which("node") is None, reason="node not installed")


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_cpuref_js_matches_golden(case):
    with tempfile.TemporaryDirectory() as d:
        inp, out = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        with open(inp, "wb") as f:
            f.write(case["x"].tobytes())
            f.write(case["blob"].tobytes())
        subprocess.check_call(["node", os.path.join(ROOT, "oracle", "cpuref.js"), case["fmt"], str(case["M"]),
                               str(case["K"]), str(case["N"]), inp, out], stdout=subprocess.DEVNULL)
        y = np.fromfile(out, dtype=np.float32)
    assert np.array_equal(y, case["y"])
