"""Writes the small golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference holds no golden vectors (all its tests draw from unseeded Math.random), so these
are produced by this repo's CPU oracle on seeded inputs shaped like the reference's own
selfValidate gates (src/lib/webgpu/kernels.ts:2325-2459): x and W uniform in [-1, 1), W passed
through the reference's quantizer (restated in oracle.quantize_q*), then
y = f32(sum x * deq(W)) with an f64 running sum. They are regression vectors; what pins the oracle
itself is tests/test_oracle_*.py.

Format: golden.json lists each case (fmt, M, K, N, plus byte offsets into golden.bin of x, the packed
.brik blob, y and deq), so both numpy and the JavaScript tests can read it.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402
from brimkern_amd import synth, layout  # noqa: E402

CASES = [
    # (fmt, M, K, N): the reference's gate shapes (m=1/5/20, k=128, n=6/18) plus odd sizes
    ("q4", 1, 128, 6), ("q4", 5, 128, 6), ("q4", 20, 128, 18), ("q4", 3, 96, 37),
    ("q8", 1, 128, 6), ("q8", 5, 128, 6), ("q8", 20, 128, 18), ("q8", 2, 224, 33),
    ("q3", 1, 128, 6), ("q3", 5, 128, 6), ("q3", 20, 128, 18), ("q3", 4, 64, 41),
]
MOE = {"E": 4, "K": 64, "N": 48, "row_off": [0, 3, 3, 11, 14]}


def quantize(fmt, W):
    if fmt == "q8":
        c, s = O.quantize_q8(W)
        return {"codes": c, "sc": s}, O.dequant_q8(c, s)
    if fmt == "q4":
        nb, s, m = O.quantize_q4(W)
        return {"nib": nb, "sc": s, "mn": m}, O.dequant_q4(nb, s, m)
    lo, hi, s, m = O.quantize_q3(W)
    return {"lo": lo, "hi": hi, "sc": s, "mn": m}, O.dequant_q3(lo, hi, s, m)


def main():
    blobs, entries = [], []
    off = 0

    def put(arr):
        nonlocal off
        b = np.ascontiguousarray(arr).view(np.uint8).ravel()
        pad = (-off) % 16
        if pad:
            blobs.append(np.zeros(pad, np.uint8))
            off += pad
        start = off
        blobs.append(b)
        off += b.size
        return [start, int(b.size)]

    for i, (fmt, M, K, N) in enumerate(CASES):
        x = synth.uniform(1000 + i, M * K, -1.0, 1.0).astype(np.float32)
        W = synth.uniform(2000 + i, N * K, -1.0, 1.0).astype(np.float32)
        planes, deq = quantize(fmt, W)
        blob = layout.pack(fmt, planes)
        y = {"q8": O.matmul_t_q8, "q4": O.matmul_t_q4, "q3": O.matmul_t_q3}[fmt](
            x, *[planes[k] for k in {"q8": ("codes", "sc"), "q4": ("nib", "sc", "mn"),
                                     "q3": ("lo", "hi", "sc", "mn")}[fmt]], M, K, N)
        entries.append({"name": f"{fmt}_m{M}_k{K}_n{N}", "fmt": fmt, "M": M, "K": K, "N": N,
                        "x": put(x), "blob": put(blob), "y": put(y), "deq": put(deq)})

    E, K, N, ro = MOE["E"], MOE["K"], MOE["N"], np.array(MOE["row_off"], np.int32)
    R = int(ro[-1])
    x = synth.uniform(3000, R * K, -1.0, 1.0).astype(np.float32)
    W = synth.uniform(3001, E * N * K, -1.0, 1.0).astype(np.float32)
    planes, _ = quantize("q4", W)
    y = O.moe_matmul_t_q4(x, ro, planes["nib"], planes["sc"], planes["mn"], E, K, N)
    moe = {"name": "moe_q4", "E": E, "K": K, "N": N, "R": R, "row_off": MOE["row_off"],
           "x": put(x), "blob": put(layout.pack("q4", planes)), "y": put(y)}

    with open(os.path.join(HERE, "golden.bin"), "wb") as f:
        f.write(np.concatenate(blobs).tobytes())
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": entries, "moe": moe}, f, indent=1)
    print(f"wrote {len(entries)} cases + moe, {off} bytes")


if __name__ == "__main__":
    main()
