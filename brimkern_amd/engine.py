"""Host-side mirror of the reference engine's quantized-matmul interface (Python host).

Mirrors the subset of ``WebGpuEngine`` (``src/lib/webgpu/kernels.ts``) that the quantized matmul
path exposes, with the same names, argument meaning and error behaviour, over ``libbrik.so``:

=========================  ===================================================  ==================
reference                  here                                                 reference lines
=========================  ===================================================  ==================
``uploadGpuRaw(bytes)``    :meth:`Engine.upload_gpu_raw` (pads to 4 bytes)       kernels.ts:1032-1042
``matmulQ4(a,nib,sc,mn,    :meth:`Engine.matmul_q4` (+ ``_tiled``/``_shared``)   kernels.ts:1046-1075
m,k,n)``
``matmulQ8(a,codes,sc,     :meth:`Engine.matmul_q8` (+ ``_tiled``/``_shared``)   kernels.ts:1140-1169
m,k,n)``
``matmulQ3(a,lo,hi,sc,mn,  :meth:`Engine.matmul_q3`                              kernels.ts:1080-1087
m,k,n)``
``dequantGpuQ4/Q3/Q8``     :meth:`Engine.weight` (one upload, planes in place)   model.ts:214-270
``recMM(enc,trash,a,w,     :meth:`Engine.mm` (dispatch on the handle's shape)    kernels.ts:1562-1567
m,k,n)``
``decodeTopKQ8`` head      :meth:`Engine.lm_head_top_k` (LM head + softcap +     kernels.ts:1934-1968
+ sampling passes          penalty + top-k, ``{ids, vals}`` sorted descending)
softcap/penalize/top_k     :meth:`Engine.logits_top_k` (on device logits)        kernels.ts:1940-1958
``quantizeToBytes(type,    :meth:`Engine.quantize_to_bytes` (GPU encode, bytes   kernels.ts:281-331
data,n,dtype)``            equal to the CPU ``encodeTensor``)
``f32ToQ8Gpu/f32ToQ4Gpu``  :meth:`Engine.quantize` (device f32 -> handle)        kernels.ts:986-1010
``matmulT(a,w,m,k,n,      :meth:`Engine.matmul_t_f16w` (f16 weight bits)       kernels.ts:410-426,
wF16)``                    (MATMUL_T_F16W)                                      shaders.ts:2240-2259
session ``conv2d`` with a  :meth:`Engine.conv2d` (q8 / q4 handle)              kernels.ts:1233-1256,
q8 / q4 weight                                                                  1369-1374
.brik container            :mod:`brimkern_amd.container`,                        container.ts:30-87
                           :meth:`Engine.weight_from_container`
=========================  ===================================================  ==================

The readback ops take host ``float32`` activations and return a host ``float32`` array of
``m*n`` (the reference returns ``Promise<Float32Array>``). The reference validates nothing and lets
WebGPU fail silently; here invalid shapes raise :class:`~brimkern_amd.capi.BrikError` before any
launch. The ``_tiled``/``_shared`` variants exist in the reference only to pick a kernel by M; here
one entry point picks the MI355X kernel by M, so they are aliases with the same output contract.
"""
from __future__ import annotations

import numpy as np

from . import container, layout
from .capi import BrikError, Context, DeviceBuffer, BRIK_EINVAL


class QWeight(dict):
    """A quantized weight handle: ``{nib, sc, mn}`` (q4), ``{codes, sc}`` (q8) or
    ``{q3: True, lo, hi, sc, mn}`` (q3) of device addresses, like ``model.ts:214-270`` builds."""

    @property
    def fmt(self) -> str:
        return "q3" if self.get("q3") else "q4" if "nib" in self else "q8"


class Engine:
    def __init__(self, device: int = 0, ctx: Context | None = None):
        """An engine on HIP device ``device``, or over an existing context ``ctx`` (not closed by
        :meth:`close`)."""
        self._own = ctx is None
        self.ctx = Context(device) if ctx is None else ctx

    def close(self):
        if self._own:
            self.ctx.close()

    # ---- uploads ---------------------------------------------------------------------
    def upload_gpu_raw(self, data) -> DeviceBuffer:
        """Persistent device copy of raw bytes, padded to a 4-byte multiple (kernels.ts:1032-1042)."""
        b = np.frombuffer(memoryview(np.ascontiguousarray(data)).cast("B"), dtype=np.uint8)
        pad = (-b.size) % 4
        if pad:
            b = np.concatenate([b, np.zeros(pad, np.uint8)])
        return self.ctx.upload(b)

    def weight(self, fmt: str, blob, n_elems: int) -> QWeight:
        """Upload a packed .brik blob once and address its planes in place."""
        offs = layout.plane_offsets(fmt, n_elems)
        buf = self.upload_gpu_raw(np.asarray(blob, np.uint8)[: layout.byte_length(fmt, n_elems)])
        h = QWeight({k: buf.offset(o) for k, (o, _) in offs.items()})
        if fmt == "q3":
            h["q3"] = True
        h["_buf"] = buf
        return h

    # ---- encoding -------------------------------------------------------------------------
    _PLANES = {"q8": ("codes", "sc"), "q4": ("nib", "sc", "mn"), "q3": ("lo", "hi", "sc", "mn")}
    # bytes of each plane per element
    _PER_ELEM = {"codes": 1.0, "nib": 0.5, "lo": 0.25, "hi": 0.125, "sc": 1 / 16, "mn": 1 / 16}

    def quantize(self, dtype: str, src, n_elems: int) -> QWeight:
        """``f32ToQ8Gpu`` / ``f32ToQ4Gpu`` (kernels.ts:986-1010) and the q3 analogue: ``n_elems`` f32
        values at device address ``src`` -> a weight handle (one buffer in packQ* layout), with the
        bytes of the CPU encoder quantizeQ*."""
        if dtype not in self._PLANES:
            raise BrikError(BRIK_EINVAL, f"quantize: unknown dtype {dtype!r}")
        offs = layout.plane_offsets(dtype, n_elems)
        buf = self.ctx.alloc(max(layout.byte_length(dtype, n_elems), 1))
        h = QWeight({k: buf.offset(o) for k, (o, _) in offs.items()})
        try:
            self.ctx.quantize(dtype, src, [h[p] for p in self._PLANES[dtype]], n_elems)
        except BrikError:
            self.ctx.free(buf)
            raise
        if dtype == "q3":
            h["q3"] = True
        h["_buf"] = buf
        return h

    def quantize_to_bytes(self, type_: str, data, n_elems: int, dtype: str, chunk: int | None = None) -> np.ndarray:
        """``quantizeToBytes`` (kernels.ts:281-331): tensor bytes -> packed .brik bytes (uint8), encoded
        on the GPU chunk by chunk and read back; equal to the CPU ``encodeTensor`` bytes (codec.ts:17-29).
        ``type_``: 'F32', 'F16' (decoded as kernels.ts:3213-3222 does) or 'Q8W' / 'Q4W' / 'Q3W' (a packed
        .brik quant, dequantized on the GPU). ``chunk`` elements per pass (default 2^26), rounded to
        whole groups (512 elements for quant sources); every chunking gives the same bytes."""
        if dtype not in self._PLANES:
            raise BrikError(BRIK_EINVAL, f"quantize_to_bytes: unknown dtype {dtype!r}")
        if n_elems < 0 or n_elems % 32:
            raise BrikError(BRIK_EINVAL, f"quantize_to_bytes: nElems {n_elems} is not a multiple of 32")
        src = np.frombuffer(memoryview(np.ascontiguousarray(data)).cast("B"), np.uint8)
        qsrc = {"Q8W": "q8", "Q4W": "q4", "Q3W": "q3"}.get(type_)
        need = {"F32": 4 * n_elems, "F16": 2 * n_elems}.get(type_)
        if need is None and qsrc:
            need = layout.byte_length(qsrc, n_elems)
        if need is None:
            raise BrikError(BRIK_EINVAL, f"quantize_to_bytes: unsupported source type {type_!r}")
        if src.size < need:
            raise BrikError(BRIK_EINVAL, f"quantize_to_bytes: {type_} data has {src.size} bytes, need {need}")
        out = np.zeros(layout.byte_length(dtype, n_elems), np.uint8)
        if n_elems == 0:
            return out
        unit = 512 if qsrc else 32
        ch = (1 << 26) if chunk is None else int(chunk)
        ch = min(max(unit, ch // unit * unit), n_elems)
        out_offs = layout.plane_offsets(dtype, n_elems)
        cap = -(-ch // 32) * 32
        ch_offs = layout.plane_offsets(dtype, cap)
        f32 = self.ctx.alloc(4 * ch)
        qbuf = self.ctx.alloc(layout.byte_length(dtype, cap))
        stage = self.ctx.alloc(2 * ch) if type_ == "F16" else None
        w = self.weight(qsrc, src, n_elems) if qsrc else None
        pe = self._PER_ELEM
        try:
            for e0 in range(0, n_elems, ch):
                ce = min(ch, n_elems - e0)
                if type_ == "F32":
                    self.ctx.h2d(f32, src[4 * e0:4 * (e0 + ce)])
                elif type_ == "F16":
                    self.ctx.h2d(stage, src[2 * e0:2 * (e0 + ce)])
                    self.ctx.f16_to_f32(stage, f32, ce)
                else:
                    at = {p: w[p] + int(e0 * pe[p]) for p in self._PLANES[qsrc]}
                    getattr(self.ctx, f"dequant_{qsrc}")(*[at[p] for p in self._PLANES[qsrc]], f32, ce)
                dst = {p: qbuf.offset(ch_offs[p][0]) for p in self._PLANES[dtype]}
                self.ctx.quantize(dtype, f32, [dst[p] for p in self._PLANES[dtype]], ce)
                for p in self._PLANES[dtype]:
                    ln, o = int(ce * pe[p]), out_offs[p][0] + int(e0 * pe[p])
                    out[o:o + ln] = self.ctx.download(dst[p], np.uint8, ln)
        finally:
            self.ctx.free(f32)
            self.ctx.free(qbuf)
            if stage is not None:
                self.ctx.free(stage)
            if w is not None:
                self.ctx.free(w["_buf"])
        return out

    def conv2d(self, inp, w: QWeight, bias, Cin: int, H: int, W: int, Cout: int, kh: int, kw: int,
               stride: int = 1, pad: int = 0, out=None) -> DeviceBuffer:
        """The recording session's conv2d for a q8 / q4 weight handle (kernels.ts:1369-1374, fused-dequant
        conv2d_direct_q8 / q4): ``inp`` [Cin, H, W] and ``bias`` [Cout] (or None) are device buffers or
        host float32 arrays; returns the device buffer ``out`` [Cout, OH, OW]."""
        fmt = w.fmt
        if fmt == "q3":
            raise BrikError(BRIK_EINVAL, "conv2d: the weight must be a q8 or q4 handle")
        OH, OW = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
        tmp = []

        def dev(v):
            if v is None or isinstance(v, (DeviceBuffer, int)):
                return v
            b = self.ctx.upload(np.ascontiguousarray(v, np.float32).ravel())
            tmp.append(b)
            return b
        y = out if out is not None else self.ctx.alloc(max(Cout * OH * OW, 1) * 4)
        planes = (w["codes"], w["sc"]) if fmt == "q8" else (w["nib"], w["sc"], w["mn"])
        try:
            self.ctx.conv2d(fmt, dev(inp), planes, dev(bias), y, Cin, H, W, Cout, kh, kw, stride, pad)
        except BrikError:
            if out is None:
                self.ctx.free(y)
            raise
        finally:
            for b in tmp:
                self.ctx.free(b)
        return y

    def weight_from_container(self, parsed: dict, name: str) -> QWeight:
        """A weight handle for tensor ``name`` of a parsed .brik file (:func:`container.parse_brik`)."""
        entry, b = container.tensor_bytes(parsed, name)
        if entry["dtype"] not in self._PLANES:
            raise BrikError(BRIK_EINVAL, f"weight_from_container: {name} has dtype {entry['dtype']}, not q8/q4/q3")
        return self.weight(entry["dtype"], np.frombuffer(b, np.uint8), entry["nElems"])

    # ---- readback ops ------------------------------------------------------------------
    def _run(self, fn, a, planes, m, k, n):
        a = np.ascontiguousarray(a, dtype=np.float32).ravel()
        if a.size != m * k:
            raise BrikError(BRIK_EINVAL, f"activation has {a.size} floats, expected m*k={m * k}")
        xa = self.ctx.upload(a) if a.size else None
        out = self.ctx.alloc(max(m * n, 1) * 4)
        try:
            fn(xa, *planes, out, m, k, n)
            res = self.ctx.download(out, np.float32, m * n)
        finally:
            self.ctx.free(out)
            if xa is not None:
                self.ctx.free(xa)
        return res

    def matmul_q4(self, a, nib, sc, mn, m, k, n) -> np.ndarray:
        return self._run(self.ctx.matmul_t_q4, a, (nib, sc, mn), m, k, n)

    matmul_q4_tiled = matmul_q4
    matmul_q4_shared = matmul_q4

    def matmul_q8(self, a, codes, sc, m, k, n) -> np.ndarray:
        return self._run(self.ctx.matmul_t_q8, a, (codes, sc), m, k, n)

    matmul_q8_tiled = matmul_q8
    matmul_q8_shared = matmul_q8

    def matmul_t_f16w(self, a, w, m, k, n) -> np.ndarray:
        """``matmulT(a, w, m, k, n, wF16=true)`` (kernels.ts:410-426 -> MATMUL_T_F16W): ``w`` is a device
        buffer / address of N x K IEEE f16 bits; returns host float32 [m*n]."""
        return self._run(lambda xa, wb, out, M, K, N: self.ctx.matmul_t_f16w(xa, wb, out, M, K, N), a, (w,), m, k, n)

    def matmul_q3(self, a, lo, hi, sc, mn, m, k, n) -> np.ndarray:
        return self._run(self.ctx.matmul_t_q3, a, (lo, hi, sc, mn), m, k, n)

    # ---- recorded form ------------------------------------------------------------------
    def mm(self, a, w: QWeight, m: int, k: int, n: int, out=None) -> DeviceBuffer:
        """Device-resident ``recMM``: ``a`` and the result are device buffers; the kernel follows
        the handle's shape (q3 flag, nib, codes) as kernels.ts:1562-1567 does."""
        if out is None:
            out = self.ctx.alloc(max(m * n, 1) * 4)
        if w.get("q3"):
            self.ctx.matmul_t_q3(a, w["lo"], w["hi"], w["sc"], w["mn"], out, m, k, n)
        elif "nib" in w:
            self.ctx.matmul_t_q4(a, w["nib"], w["sc"], w["mn"], out, m, k, n)
        elif "codes" in w:
            self.ctx.matmul_t_q8(a, w["codes"], w["sc"], out, m, k, n)
        else:
            raise BrikError(BRIK_EINVAL, "mm: weight handle is not a q3/q4/q8 handle (f32/f16 weights are "
                                         "outside this library)")
        return out

    # ---- sampling pre-work ---------------------------------------------------------------
    def _top_k(self, run, recent, k):
        ids = list(dict.fromkeys(int(i) for i in (recent or [])))      # each id once, as the callers pass them
        rb = self.ctx.upload(np.asarray(ids, np.int32)) if ids else None
        ob = self.ctx.alloc(8 * k)
        try:
            run(rb, len(ids), ob, ob.offset(4 * k))
            out_ids = self.ctx.download(ob, np.int32, k).astype(np.uint32)
            out_vals = self.ctx.download(ob, np.float32, k, src_offset=4 * k)
        finally:
            self.ctx.free(ob)
            if rb is not None:
                self.ctx.free(rb)
        return out_ids, out_vals

    def logits_top_k(self, logits: DeviceBuffer, vocab: int, recent=(), penalty: float = 1.0,
                     softcap: float = 0.0, k: int = 64):
        """The passes decodeTopKQ8 records after the head (kernels.ts:1940-1958) on a device logits
        buffer, modified in place like the reference: softcap, repetition penalty, then the top ``k``.
        Returns ``(ids uint32[k], vals float32[k])`` sorted descending."""
        def run(rb, nr, ids, vals):
            self.ctx.logits_topk(logits, vocab, rb, nr, penalty, softcap, k, ids, vals)
        return self._top_k(run, recent, k)

    def lm_head_top_k(self, x, w: QWeight, d: int, vocab: int, recent=(), penalty: float = 1.0,
                      softcap: float = 0.0, k: int = 64):
        """``decodeTopKQ8``'s projection and sampling pre-work (kernels.ts:1934-1968) for one
        activation row ``x`` (host float32 [d] or a device buffer): logits = x . deq(W)^T over the
        vocab in one launch, then the passes of :meth:`logits_top_k`. Returns ``(ids, vals)``."""
        xa = x if isinstance(x, DeviceBuffer) else self.ctx.upload(np.ascontiguousarray(x, np.float32).ravel())
        fmt = w.fmt
        planes = {"q8": ("codes", "sc"), "q4": ("nib", "sc", "mn"), "q3": ("lo", "hi", "sc", "mn")}[fmt]

        def run(rb, nr, ids, vals):
            self.ctx.lm_head_topk(fmt, xa, [w[p] for p in planes], d, vocab, rb, nr, penalty, softcap, k, ids, vals)
        try:
            return self._top_k(run, recent, k)
        finally:
            if xa is not x:
                self.ctx.free(xa)
