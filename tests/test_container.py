"""The .brik container (brimkern_amd/container.py and brimkern_amd/js/container.js) on the CPU.

Mirrors the reference's container test (src/lib/brik/container.test.ts): header parse, 16-byte
aligned data section, manifest round trip, file size = dataStart + shard bytes, every tensor read back
from dataStart + shardBase + offset, bad magic rejected; plus the truncation errors of
parseBrikHeader (container.ts:72-77) and byte identity of the files the Python and JavaScript writers
produce for the same input (the manifest JSON as JSON.stringify writes it).
"""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import oracle as O
from brimkern_amd import container as C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")

ARCH = {"arch": "qwen2", "d": 64, "nHeads": 4, "nKvHeads": 2, "headDim": 16, "ffn": 128, "blockCount": 2,
        "ropeTheta": 1000000.0, "rmsEps": 1e-06, "vocab": 96}
MODEL = {"name": "synthetic", "quantSource": "test", "uiArch": "qwen"}
CHAT = {"template": "{{x}}", "stopTokenIds": [2]}
TOK = {"kind": "hf-hub", "id": "Xenova/qwen-tokenizer"}


def inputs():
    """Packed tensors of a tiny two-block model: q4 / q8 / q3 matrices (oracle-encoded), f32 norms."""
    rng = np.random.default_rng(11)
    d, ffn, vocab = ARCH["d"], ARCH["ffn"], ARCH["vocab"]
    out = []

    def q(name, fmt, shape):
        x = rng.standard_normal(int(np.prod(shape))).astype(np.float32)
        b = getattr(O, f"pack_{fmt}")(*getattr(O, f"quantize_{fmt}")(x))
        out.append({"name": name, "dtype": fmt, "shape": list(shape), "bytes": b.tobytes(), "nElems": x.size,
                    "_x": x})

    def f(name, n):
        x = rng.standard_normal(n).astype(np.float32)
        out.append({"name": name, "dtype": "f32", "shape": [n], "data": x, "_x": x})

    q("token_embd.weight", "q4", (vocab, d))
    f("output_norm.weight", d)
    for i in range(2):
        f(f"blk.{i}.attn_norm.weight", d)
        q(f"blk.{i}.attn_q.weight", "q8", (d, d))
        q(f"blk.{i}.ffn_down.weight", "q3", (d, ffn))
    return out


def build():
    ts = inputs()
    manifest, shards = C.assemble_brik(MODEL, ARCH, CHAT, TOK, [{k: v for k, v in t.items() if k != "_x"}
                                                                for t in ts])
    return ts, manifest, shards, C.serialize_brik(manifest, shards)


def test_header_and_layout():
    ts, manifest, shards, f = build()
    h = C.parse_brik_header(f)
    assert f[:4] == b"BRIK" and h["version"] == C.BRIK_VERSION == 1
    assert h["dataStart"] % C.BRIK_ALIGN == 0
    assert len(h["manifest"]["tensors"]) == len(ts)
    assert h["manifest"]["arch"]["d"] == ARCH["d"] and h["manifest"]["tokenizer"]["id"] == TOK["id"]
    mlen = struct.unpack_from("<I", f, 8)[0]
    assert len(f) == C.brik_data_start(mlen) + sum(s["byteLength"] for s in manifest["shards"])
    # shard 0 holds the non-block tensors, then one shard per block in order
    files = [s["file"] for s in h["manifest"]["shards"]]
    assert files == ["shard-0000.brik", "shard-0001.brik", "shard-0002.brik"]
    assert h["manifest"]["tensors"]["token_embd.weight"]["shard"] == 0
    assert h["manifest"]["tensors"]["blk.1.attn_q.weight"]["shard"] == 2


def test_every_tensor_reads_back_from_its_absolute_offset():
    ts, _, _, f = build()
    p = C.parse_brik(f)
    bases = C.compute_shard_bases(p["manifest"]["shards"])
    for t in ts:
        e, b = C.tensor_bytes(p, t["name"])
        assert (p["dataStart"] + bases[e["shard"]] + e["offset"]) % C.BRIK_ALIGN == 0
        if t["dtype"] == "f32":
            assert np.array_equal(np.frombuffer(b, "<f4"), t["_x"])
        else:
            assert bytes(b) == t["bytes"]
            assert e["byteLength"] == len(t["bytes"]) and e["nElems"] == t["nElems"]


def test_rejects_bad_magic_and_truncation():
    _, manifest, _, f = build()
    bad = bytearray(f)
    bad[0] = 0
    with pytest.raises(C.BrikFormatError, match="sceau magique absent"):
        C.parse_brik_header(bytes(bad))
    with pytest.raises(C.BrikFormatError, match="tronqué \\(en-tête\\)"):
        C.parse_brik_header(f[:11])
    mlen = struct.unpack_from("<I", f, 8)[0]
    with pytest.raises(C.BrikFormatError, match="manifeste tronqué"):
        C.parse_brik_header(f[:12 + mlen - 1])
    C.parse_brik_header(f[:12 + mlen])                 # the header alone is enough
    with pytest.raises(C.BrikFormatError, match="tenseur tronqué"):
        C.tensor_bytes(C.parse_brik(f[:len(f) - 40]), "blk.1.ffn_down.weight")


def test_serialize_rejects_missing_or_resized_shards():
    _, manifest, shards, _ = build()
    with pytest.raises(C.BrikFormatError, match="shard manquant"):
        C.serialize_brik(manifest, shards[1:])
    wrong = [dict(s) for s in shards]
    wrong[1]["bytes"] = wrong[1]["bytes"] + b"\0" * 16
    with pytest.raises(C.BrikFormatError, match="taille de shard incohérente"):
        C.serialize_brik(manifest, wrong)


@pytest.mark.parametrize("v", [0, 1, -3, 7.0, 0.5, 1e-06, 1e-07, 1.5e-07, 123.456, 1e21, 1.5e21, 1e20, -2.5e-8,
                               1000000.0, 0.1 + 0.2, 5e-324, 1.7976931348623157e308, 2 ** 53 + 2.0])
def test_js_number_format(v):
    if NODE is None:
        pytest.skip("node not installed")
    r = subprocess.run([NODE, "-e", f"process.stdout.write(JSON.stringify({v!r}))"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert C._js_number(v) == r.stdout


@pytest.mark.skipif(NODE is None, reason="node not installed")
def test_python_and_js_writers_agree(tmp_path):
    ts, manifest, _, f = build()
    spec = {"model": MODEL, "arch": ARCH, "chat": dict(CHAT, template="é \"q\" \\ \n\t\u0001"), "tokenizer": TOK,
            "tensors": []}
    blobs = []
    for t in ts:
        b = t["bytes"] if "bytes" in t else t["data"].tobytes()
        blobs.append(b)
        spec["tensors"].append({k: t[k] for k in ("name", "dtype", "shape")} | ({"nElems": t["nElems"]} if "nElems" in t
                                                                                else {}))
    raw = tmp_path / "blobs.bin"
    raw.write_bytes(b"".join(blobs))
    (tmp_path / "spec.json").write_text(json.dumps(spec))
    script = (
        "const c = require('./brimkern_amd/js/container'); const fs = require('fs');"
        f"const spec = JSON.parse(fs.readFileSync({json.dumps(str(tmp_path / 'spec.json'))}, 'utf8'));"
        f"const raw = fs.readFileSync({json.dumps(str(raw))}); let off = 0;"
        "const lens = " + json.dumps([len(b) for b in blobs]) + ";"
        "spec.tensors.forEach(function (t, i) { const b = new Uint8Array(raw.buffer, raw.byteOffset + off, lens[i]);"
        " off += lens[i]; if (t.dtype === 'f32') t.data = new Float32Array(b.slice().buffer); else t.bytes = b; });"
        "const o = c.assembleBrik(spec); const f = c.serializeBrik(o.manifest, o.shards);"
        f"fs.writeFileSync({json.dumps(str(tmp_path / 'js.brik'))}, Buffer.from(f));"
    )
    r = subprocess.run([NODE, "-e", script], cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    pm, ps = C.assemble_brik(MODEL, ARCH, spec["chat"], TOK, [{k: v for k, v in t.items() if k != "_x"} for t in ts])
    assert (tmp_path / "js.brik").read_bytes() == C.serialize_brik(pm, ps)
    # and the JS reader reads the Python file's tensors at the same offsets
    (tmp_path / "py.brik").write_bytes(f)
    r = subprocess.run([NODE, "-e", "const c = require('./brimkern_amd/js/container');"
                        f"const p = c.parseBrik(require('fs').readFileSync({json.dumps(str(tmp_path / 'py.brik'))}));"
                        "const o = {}; Object.keys(p.manifest.tensors).forEach(function (n) {"
                        " const t = c.tensorBytes(p, n); o[n] = [p.dataStart + (t.bytes.byteOffset - p.data.byteOffset),"
                        " t.bytes.length]; }); console.log(JSON.stringify(o));"],
                       cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    p = C.parse_brik(f)
    for name, (start, ln) in json.loads(r.stdout).items():
        e, b = C.tensor_bytes(p, name)
        assert bytes(f[start:start + ln]) == bytes(b)


def test_js_reader_and_writer_error_messages(tmp_path):
    """The JS module raises the reference's messages on the same bad inputs as the Python one."""
    if NODE is None:
        pytest.skip("node not installed")
    _, manifest, shards, f = build()
    (tmp_path / "f.brik").write_bytes(f)
    mlen = struct.unpack_from("<I", f, 8)[0]
    script = (
        "const c = require('./brimkern_amd/js/container'); const fs = require('fs');"
        f"const f = new Uint8Array(fs.readFileSync({json.dumps(str(tmp_path / 'f.brik'))}));"
        "function msg(fn) { try { fn(); return null; } catch (e) { return e.message; } }"
        "const bad = f.slice(); bad[0] = 0; const p = c.parseBrik(f);"
        "const shards = p.manifest.shards.map(function (s) { const b = c.computeShardBases(p.manifest.shards)[s.id];"
        " return { file: s.file, bytes: p.data.slice(b, b + s.byteLength) }; });"
        "const grown = shards.map(function (s, i) { return i === 1 ? { file: s.file, bytes: new Uint8Array(s.bytes.length + 16) } : s; });"
        "console.log(JSON.stringify({"
        " magic: msg(function () { c.parseBrikHeader(bad); }),"
        " header: msg(function () { c.parseBrikHeader(f.subarray(0, 11)); }),"
        f" manifest: msg(function () {{ c.parseBrikHeader(f.subarray(0, {12 + mlen - 1})); }}),"
        f" headerOnly: msg(function () {{ c.parseBrikHeader(f.subarray(0, {12 + mlen})); }}),"
        " tensorCut: msg(function () { c.tensorBytes(c.parseBrik(f.subarray(0, f.length - 40)), 'blk.1.ffn_down.weight'); }),"
        " tensorGone: msg(function () { c.tensorBytes(p, 'nope'); }),"
        " missing: msg(function () { c.serializeBrik(p.manifest, shards.slice(1)); }),"
        " resized: msg(function () { c.serializeBrik(p.manifest, grown); }),"
        " roundTrip: Buffer.from(c.serializeBrik(p.manifest, shards)).equals(Buffer.from(f)) }));"
    )
    r = subprocess.run([NODE, "-e", script], cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    m = json.loads(r.stdout)
    assert m["magic"].startswith("BRIK: sceau magique absent (")
    assert m["header"] == "BRIK: fichier tronqué (en-tête)"
    assert m["manifest"] == "BRIK: manifeste tronqué"
    assert m["headerOnly"] is None
    assert m["tensorCut"] == "BRIK: tenseur tronqué : blk.1.ffn_down.weight"
    assert m["tensorGone"] == "BRIK: tenseur absent : nope"
    assert m["missing"] == f"shard manquant : {manifest['shards'][0]['file']}"
    s1 = manifest["shards"][1]
    assert m["resized"] == f"taille de shard incohérente pour {s1['file']} : {s1['byteLength'] + 16} ≠ {s1['byteLength']}"
    assert m["roundTrip"] is True
