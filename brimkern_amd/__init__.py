"""brimkern_amd — MI355X (gfx950) drop-in for Brimkern's fused quantized matmuls.

``matmul_t_q8`` / ``matmul_t_q4`` / ``matmul_t_q3``: ``y[M,N] = x[M,K] . deq(W[N,K])^T`` over the
exact ``.brik`` planes, as hand-written HIP kernels in ``libbrik.so`` (C ABI: ``include/brik.h``).
Hosts: ``brimkern_amd.engine`` (Python, ctypes) and ``brimkern_amd/js`` (Node, N-API).
"""
from .capi import BrikError, Context, DeviceBuffer, load_library, device_count  # noqa: F401
from .engine import Engine, QWeight  # noqa: F401
from . import layout, synth  # noqa: F401

__all__ = ["BrikError", "Context", "DeviceBuffer", "Engine", "QWeight", "load_library", "device_count",
           "layout", "synth"]
