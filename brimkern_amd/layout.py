""".brik quantized tensor layouts: plane offsets inside one packed blob.

Same offsets as the reference's ``unpackQ8`` / ``unpackQ4`` / ``unpackQ3``
(``src/lib/brik/q8web.ts:65-72``, ``q4web.ts:70-80``, ``q3web.ts:80-95``) and byte lengths as
``q8ByteLength`` / ``q4ByteLength`` / ``q3ByteLength`` (``q8web.ts:23-26``, ``q4web.ts:23-26``,
``q3web.ts:29-32``). The reference copies each plane into its own GPU buffer
(``model.ts:214-270``); here a blob is uploaded once and the planes are addressed in place, which the
alignment contract of ``include/brik.h`` allows for any 16-byte aligned blob.
"""
from __future__ import annotations

GROUP = 32
FORMATS = ("q8", "q4", "q3")


def byte_length(fmt: str, n: int) -> int:
    g = n // GROUP
    if fmt == "q8":
        return n + 2 * g
    if fmt == "q4":
        return n // 2 + 4 * g
    if fmt == "q3":
        return (n // 16) * 4 + (n // 32) * 4 + 4 * g
    raise ValueError(fmt)


def plane_offsets(fmt: str, n: int) -> dict:
    """Byte offset and length of every plane of an ``n``-element tensor inside its packed blob."""
    if n % GROUP:
        raise ValueError(f"{fmt}: nElems={n} is not a multiple of {GROUP}")
    g = n // GROUP
    if fmt == "q8":
        return {"codes": (0, n), "sc": (n, 2 * g)}
    if fmt == "q4":
        return {"nib": (0, n // 2), "sc": (n // 2, 2 * g), "mn": (n // 2 + 2 * g, 2 * g)}
    if fmt == "q3":
        lb, hb = (n // 16) * 4, (n // 32) * 4
        return {"lo": (0, lb), "hi": (lb, hb), "sc": (lb + hb, 2 * g), "mn": (lb + hb + 2 * g, 2 * g)}
    raise ValueError(fmt)


PLANE_DTYPES = {"codes": "i1", "nib": "u1", "lo": "<u4", "hi": "<u4", "sc": "<u2", "mn": "<u2"}


def split_blob(fmt: str, blob, n: int) -> dict:
    """numpy views of the planes of a packed blob (host side ``unpackQ*``)."""
    import numpy as np
    b = np.asarray(blob, dtype=np.uint8)
    if b.size < byte_length(fmt, n):
        raise ValueError(f"{fmt} blob of {b.size} bytes is shorter than {byte_length(fmt, n)}")
    return {k: b[o:o + ln].view(PLANE_DTYPES[k]) for k, (o, ln) in plane_offsets(fmt, n).items()}


def pack(fmt: str, planes: dict):
    """Concatenate planes into one blob (``packQ8`` / ``packQ4`` / ``packQ3`` order)."""
    import numpy as np
    order = {"q8": ("codes", "sc"), "q4": ("nib", "sc", "mn"), "q3": ("lo", "hi", "sc", "mn")}[fmt]
    return np.concatenate([np.ascontiguousarray(planes[k], dtype=PLANE_DTYPES[k]).view(np.uint8) for k in order])
