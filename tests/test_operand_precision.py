"""Why the MFMA GEMM multiplies f16 operands, not bf16: the 1e-3 normwise bar measured on the CPU.

The GEMM stages each activation row scaled by a power of two and rounded to f16, and dequantizes each
weight to f16 (q s + m rounded once); products accumulate in f32. Emulating that on q4 weights of the
prefill shapes (accumulation in f64, so only the operand rounding shows) gives a normwise error near
3e-4 against the oracle. The same with both operands rounded to bf16 (8-bit significand, round to
nearest even) gives 2e-3 to 3e-3, over the bar.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth


def to_bf16(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("M,K,N,seed", [(64, 2560, 512, 1), (32, 9728, 256, 3)])
def test_f16_operands_pass_and_bf16_would_not(M, K, N, seed):
    t = synth.q4_tensor(seed, N, K)
    x = synth.normal(seed + 10, M * K).reshape(M, K)
    w = O.dequant_q4(t["nib"], t["sc"], t["mn"]).reshape(N, K)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    e = np.floor(np.log2(np.abs(x).max(axis=1, keepdims=True)))
    xf16 = (x * 2.0 ** (15 - e)).astype(np.float16).astype(np.float64) * 2.0 ** (e - 15)
    y_f16 = xf16 @ w.astype(np.float16).astype(np.float64).T
    y_bf16 = to_bf16(x).astype(np.float64) @ to_bf16(w).astype(np.float64).T

    def normwise(y):
        return np.abs(y - ref).max() / np.abs(ref).max()
    assert normwise(y_f16) < 5e-4
    assert normwise(y_bf16) > 1.5e-3
