"""The single-file .brik container and its shard layout (Python side of ``js/container.js``).

Same layout, offsets and error messages as the reference's ``src/lib/brik/container.ts``
(``serializeBrik`` :30-58, ``parseBrikHeader`` :71-81, ``parseBrik`` :84-87), ``codec.ts:62-98``
(``packShard``), ``convert.ts:37-89`` (``assembleBrik``, shard grouping) and ``loader.ts:57-66``
(``computeShardBases``)::

    [0, 4)        magic "BRIK"
    [4, 8)        version, u32 LE (1)
    [8, 12)       manifest byte length L, u32 LE
    [12, 12 + L)  manifest JSON (UTF-8)
    [alignUp(12 + L, 16), ...)  shard bytes in ascending shard-id order

The manifest is written as ``JSON.stringify`` writes it (no spaces, numbers in ECMAScript's
shortest form), so a file written here is byte-identical to the reference's for the same manifest
and shards. Quantized tensors are stored as packed planes (``packQ*`` bytes), produced on the GPU by
:meth:`brimkern_amd.engine.Engine.quantize_to_bytes`.
"""
from __future__ import annotations

import json
import math
import re
import struct

BRIK_VERSION = 1      # format.ts:6
BRIK_ALIGN = 16       # format.ts:8
MAGIC = b"BRIK"
HEADER_FIXED = 12


class BrikFormatError(ValueError):
    pass


def align_up(n: int, align: int = BRIK_ALIGN) -> int:
    return -(-n // align) * align


def brik_data_start(manifest_byte_length: int) -> int:
    return align_up(HEADER_FIXED + manifest_byte_length)


def _js_number(x) -> str:
    """ECMAScript Number::toString for a finite number (JSON.stringify writes null otherwise)."""
    if isinstance(x, bool):
        return "true" if x else "false"
    if isinstance(x, int) and abs(x) < 2 ** 53:
        return str(x)
    f = float(x)
    if not math.isfinite(f):
        return "null"
    if f == 0:
        return "0"
    sign = "-" if f < 0 else ""
    mant, _, exp = repr(abs(f)).partition("e")
    ip, _, fp = mant.partition(".")
    digits = (ip + fp).lstrip("0")
    # decimal exponent n: value = 0.d1d2... x 10^n
    n = len(ip.lstrip("0")) if ip.strip("0") else -(len(fp) - len(fp.lstrip("0")))
    n += int(exp) if exp else 0
    digits = digits.rstrip("0") or "0"
    k = len(digits)
    if k <= n <= 21:
        s = digits + "0" * (n - k)
    elif 0 < n <= 21:
        s = digits[:n] + "." + digits[n:]
    elif -6 < n <= 0:
        s = "0." + "0" * (-n) + digits
    else:
        e = n - 1
        s = digits[0] + ("." + digits[1:] if k > 1 else "") + "e" + ("+" if e >= 0 else "-") + str(abs(e))
    return sign + s


def _js_json(v) -> str:
    """JSON.stringify(v) for the JSON value types a manifest holds."""
    if v is None:
        return "null"
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, (int, float)):
        return _js_number(v)
    if isinstance(v, str):
        return json.dumps(v, ensure_ascii=False)
    if isinstance(v, (list, tuple)):
        return "[" + ",".join(_js_json(e) for e in v) + "]"
    if isinstance(v, dict):
        return "{" + ",".join(json.dumps(str(k), ensure_ascii=False) + ":" + _js_json(e) for k, e in v.items()) + "}"
    raise TypeError(f"not JSON-serialisable: {type(v).__name__}")


def serialize_brik(manifest: dict, shards: list) -> bytes:
    """``serializeBrik``: ``shards`` is a list of ``{"file": str, "bytes": bytes-like}``."""
    mbytes = _js_json(manifest).encode("utf-8")
    data_start = brik_data_start(len(mbytes))
    ordered = sorted(manifest["shards"], key=lambda s: s["id"])
    by_file = {s["file"]: memoryview(s["bytes"]).cast("B") for s in shards}
    for sh in ordered:
        b = by_file.get(sh["file"])
        if b is None:
            raise BrikFormatError(f"shard manquant : {sh['file']}")
        if len(b) != sh["byteLength"]:
            raise BrikFormatError(f"taille de shard incohérente pour {sh['file']} : {len(b)} ≠ {sh['byteLength']}")
    out = bytearray(data_start + sum(sh["byteLength"] for sh in ordered))
    out[0:4] = MAGIC
    struct.pack_into("<II", out, 4, BRIK_VERSION, len(mbytes))
    out[HEADER_FIXED:HEADER_FIXED + len(mbytes)] = mbytes
    off = data_start
    for sh in ordered:
        out[off:off + sh["byteLength"]] = by_file[sh["file"]]
        off += sh["byteLength"]
    return bytes(out)


def parse_brik_header(data) -> dict:
    """``parseBrikHeader``: ``{"manifest", "version", "dataStart"}`` from the leading bytes."""
    b = memoryview(data).cast("B")
    if len(b) < HEADER_FIXED:
        raise BrikFormatError("BRIK: fichier tronqué (en-tête)")
    magic = bytes(b[0:4])
    if magic != MAGIC:
        raise BrikFormatError(f"BRIK: sceau magique absent ({magic.decode('latin-1')})")
    version, mlen = struct.unpack_from("<II", b, 4)
    if HEADER_FIXED + mlen > len(b):
        raise BrikFormatError("BRIK: manifeste tronqué")
    manifest = json.loads(bytes(b[HEADER_FIXED:HEADER_FIXED + mlen]).decode("utf-8"))
    return {"manifest": manifest, "version": version, "dataStart": brik_data_start(mlen)}


def parse_brik(data) -> dict:
    """``parseBrik``: the header plus ``data``, a view of the data section."""
    b = memoryview(data).cast("B")
    h = parse_brik_header(b)
    h["data"] = b[h["dataStart"]:]
    return h


def compute_shard_bases(shards: list) -> dict:
    """``computeShardBases``: shard id -> byte offset in the data section."""
    bases, off = {}, 0
    for sh in sorted(shards, key=lambda s: s["id"]):
        bases[sh["id"]] = off
        off += sh["byteLength"]
    return bases


def tensor_bytes(parsed: dict, name: str):
    """``(entry, bytes view)`` of one tensor of a parsed file."""
    e = parsed["manifest"]["tensors"].get(name)
    if e is None:
        raise BrikFormatError(f"BRIK: tenseur absent : {name}")
    base = compute_shard_bases(parsed["manifest"]["shards"]).get(e["shard"])
    if base is None or base + e["offset"] + e["byteLength"] > len(parsed["data"]):
        raise BrikFormatError(f"BRIK: tenseur tronqué : {name}")
    start = base + e["offset"]
    return e, parsed["data"][start:start + e["byteLength"]]


def pack_shard(tensors: list, shard_id: int):
    """``packShard``: ``tensors`` are ``{"name", "dtype", "shape", "bytes" | "data" (f32 only),
    "nElems"}``; each starts on a 16-byte boundary and the shard length is padded to 16."""
    import numpy as np
    enc = []
    for t in tensors:
        b = t.get("bytes")
        if b is None:
            if t["dtype"] != "f32" or t.get("data") is None:
                raise BrikFormatError(f"packShard: {t['name']} needs pre-encoded bytes for dtype {t['dtype']}")
            b = np.ascontiguousarray(t["data"], "<f4").tobytes()
        b = bytes(memoryview(b).cast("B"))
        n = t.get("nElems")
        if n is None:
            n = len(t["data"]) if t.get("data") is not None else int(np.prod(t["shape"]))
        enc.append((t, b, int(n)))
    total = 0
    for _, b, _ in enc:
        total = align_up(total) + len(b)
    buf = bytearray(align_up(total))
    entries, cursor = {}, 0
    for t, b, n in enc:
        cursor = align_up(cursor)
        buf[cursor:cursor + len(b)] = b
        entries[t["name"]] = {"dtype": t["dtype"], "shape": list(t["shape"]), "nElems": n, "shard": shard_id,
                              "offset": cursor, "byteLength": len(b)}
        cursor += len(b)
    return bytes(buf), entries


def _group_key(name: str) -> str:
    m = re.match(r"^blk\.(\d+)\.", name)
    return f"layer-{m.group(1).zfill(4)}" if m else "shared"


def _order_shard_keys(keys):
    # 'shared' first, then the rest in string order ("layer-0002" < "layer-0010")
    return sorted(keys, key=lambda k: (k != "shared", k))


def assemble_brik(model: dict, arch: dict, chat: dict, tokenizer: dict, tensors: list):
    """``assembleBrik``: one shard per transformer block (``blk.<i>.``), the rest in shard 0.
    Returns ``(manifest, shards)``."""
    groups = {}
    for t in tensors:
        groups.setdefault(_group_key(t["name"]), []).append(t)
    entries, shards, meta = {}, [], []
    for sid, key in enumerate(_order_shard_keys(groups)):
        buf, ent = pack_shard(groups[key], sid)
        entries.update(ent)
        f = f"shard-{sid:04d}.brik"
        shards.append({"file": f, "bytes": buf})
        meta.append({"id": sid, "file": f, "byteLength": len(buf)})
    manifest = {"format": "brik", "version": BRIK_VERSION, "model": model, "arch": arch, "chat": chat,
                "tokenizer": tokenizer, "shards": meta, "tensors": entries}
    return manifest, shards
