'use strict';
// The single-file .brik container and its shard layout, as the reference reads and writes them
// (src/lib/brik/container.ts, codec.ts:62-98, convert.ts:37-89, loader.ts:57-66, format.ts:6-8,
// 87-90), so that a .brik file made by either side loads in the other:
//
//   [0, 4)          magic "BRIK"
//   [4, 8)          version, u32 LE (1)
//   [8, 12)         manifest byte length L, u32 LE
//   [12, 12 + L)    manifest JSON (UTF-8)
//   [alignUp(12 + L, 16), ...)   the data section: shard bytes in ascending shard-id order
//
// A tensor's absolute file offset is dataStart + shardBase[shard] + offset; every tensor starts on a
// 16-byte boundary of its shard, and shards have 16-byte multiple lengths. Error messages keep the
// reference's text, so callers that match on them see the same errors.
//
// Quantized tensors are stored as the packed planes (packQ8 / packQ4 / packQ3 bytes); this module
// does not encode values itself: engine.quantizeToBytes (GPU) produces them.

const BRIK_VERSION = 1;
const BRIK_ALIGN = 16;
const MAGIC = 'BRIK';
const HEADER_FIXED = 12;

function alignUp(n, align) {
  const a = align === undefined ? BRIK_ALIGN : align;
  return Math.ceil(n / a) * a;
}

function brikDataStart(manifestByteLength) { return alignUp(HEADER_FIXED + manifestByteLength); }

function asBytes(data) {
  if (data instanceof Uint8Array) return data;
  if (ArrayBuffer.isView(data)) return new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
  if (data instanceof ArrayBuffer) return new Uint8Array(data);
  throw new TypeError('expected bytes (TypedArray / ArrayBuffer)');
}

// container.ts:30-58
function serializeBrik(manifest, shards) {
  const manifestBytes = Buffer.from(JSON.stringify(manifest), 'utf8');
  const dataStart = brikDataStart(manifestBytes.length);
  const ordered = manifest.shards.slice().sort(function (a, b) { return a.id - b.id; });
  const byFile = new Map(shards.map(function (s) { return [s.file, asBytes(s.bytes)]; }));
  let dataLen = 0;
  ordered.forEach(function (sh) {
    const bytes = byFile.get(sh.file);
    if (!bytes) throw new Error('shard manquant : ' + sh.file);
    if (bytes.length !== sh.byteLength) {
      throw new Error('taille de shard incohérente pour ' + sh.file + ' : ' + bytes.length + ' ≠ ' + sh.byteLength);
    }
    dataLen += sh.byteLength;
  });
  const out = new Uint8Array(dataStart + dataLen);
  for (let i = 0; i < MAGIC.length; i++) out[i] = MAGIC.charCodeAt(i);
  const dv = new DataView(out.buffer);
  dv.setUint32(4, BRIK_VERSION, true);
  dv.setUint32(8, manifestBytes.length, true);
  out.set(manifestBytes, HEADER_FIXED);
  let off = dataStart;
  ordered.forEach(function (sh) {
    out.set(byFile.get(sh.file), off);
    off += sh.byteLength;
  });
  return out;
}

// container.ts:71-81: header + manifest from the leading bytes of a file
function parseBrikHeader(data) {
  const bytes = asBytes(data);
  if (bytes.length < HEADER_FIXED) throw new Error('BRIK: fichier tronqué (en-tête)');
  const magic = String.fromCharCode(bytes[0], bytes[1], bytes[2], bytes[3]);
  if (magic !== MAGIC) throw new Error('BRIK: sceau magique absent (' + magic + ')');
  const dv = new DataView(bytes.buffer, bytes.byteOffset, bytes.byteLength);
  const version = dv.getUint32(4, true);
  const manifestLen = dv.getUint32(8, true);
  if (HEADER_FIXED + manifestLen > bytes.length) throw new Error('BRIK: manifeste tronqué');
  const text = Buffer.from(bytes.buffer, bytes.byteOffset + HEADER_FIXED, manifestLen).toString('utf8');
  return { manifest: JSON.parse(text), version: version, dataStart: brikDataStart(manifestLen) };
}

// container.ts:84-87
function parseBrik(data) {
  const bytes = asBytes(data);
  const h = parseBrikHeader(bytes);
  return { manifest: h.manifest, version: h.version, dataStart: h.dataStart, data: bytes.subarray(h.dataStart) };
}

// loader.ts:57-66: byte offset of each shard in the data section, indexed by shard id
function computeShardBases(shards) {
  const ordered = shards.slice().sort(function (a, b) { return a.id - b.id; });
  const bases = [];
  let off = 0;
  ordered.forEach(function (sh) {
    bases[sh.id] = off;
    off += sh.byteLength;
  });
  return bases;
}

// The bytes of one tensor of a parsed file (a view, no copy), with its manifest entry.
function tensorBytes(parsed, name) {
  const e = parsed.manifest.tensors[name];
  if (!e) throw new Error('BRIK: tenseur absent : ' + name);
  const base = computeShardBases(parsed.manifest.shards)[e.shard];
  const start = base + e.offset;
  if (base === undefined || start + e.byteLength > parsed.data.length) throw new Error('BRIK: tenseur tronqué : ' + name);
  return { entry: e, bytes: parsed.data.subarray(start, start + e.byteLength) };
}

// codec.ts:62-98: tensors [{name, dtype, shape, bytes | data (f32 only), nElems}] into one shard,
// each 16-byte aligned, the shard length padded to 16.
function packShard(tensors, shardId) {
  const encoded = tensors.map(function (t) {
    let bytes = t.bytes;
    if (!bytes) {
      if (t.dtype !== 'f32' || !t.data) throw new Error('packShard: ' + t.name + ' needs pre-encoded bytes for dtype ' + t.dtype);
      bytes = Float32Array.from(t.data);
    }
    bytes = asBytes(bytes);
    const nElems = t.nElems !== undefined ? t.nElems : t.data ? t.data.length
      : t.shape.reduce(function (a, b) { return a * b; }, 1);
    return { t: t, bytes: bytes, nElems: nElems };
  });
  let total = 0;
  encoded.forEach(function (e) { total = alignUp(total) + e.bytes.length; });
  const buffer = new Uint8Array(alignUp(total));
  const entries = {};
  let cursor = 0;
  encoded.forEach(function (e) {
    cursor = alignUp(cursor);
    buffer.set(e.bytes, cursor);
    entries[e.t.name] = { dtype: e.t.dtype, shape: e.t.shape, nElems: e.nElems, shard: shardId, offset: cursor,
      byteLength: e.bytes.length };
    cursor += e.bytes.length;
  });
  return { buffer: buffer, entries: entries };
}

// convert.ts:37-52: one shard per transformer block ("blk.<i>."), everything else in shard 0
function shardFile(id) { return 'shard-' + String(id).padStart(4, '0') + '.brik'; }
function groupKey(name) {
  const m = /^blk\.(\d+)\./.exec(name);
  return m ? 'layer-' + m[1].padStart(4, '0') : 'shared';
}
function orderShardKeys(keys) {
  return keys.slice().sort(function (a, b) { return a === 'shared' ? -1 : b === 'shared' ? 1 : a.localeCompare(b); });
}

// convert.ts:54-89: {model, arch, chat, tokenizer, tensors} -> {manifest, shards}
function assembleBrik(input) {
  const groups = new Map();
  input.tensors.forEach(function (t) {
    const k = groupKey(t.name);
    if (!groups.has(k)) groups.set(k, []);
    groups.get(k).push(t);
  });
  const tensors = {};
  const shards = [];
  const shardMeta = [];
  orderShardKeys(Array.from(groups.keys())).forEach(function (key, shardId) {
    const packed = packShard(groups.get(key), shardId);
    Object.assign(tensors, packed.entries);
    const file = shardFile(shardId);
    shards.push({ file: file, bytes: packed.buffer });
    shardMeta.push({ id: shardId, file: file, byteLength: packed.buffer.length });
  });
  const manifest = { format: 'brik', version: BRIK_VERSION, model: input.model, arch: input.arch, chat: input.chat,
    tokenizer: input.tokenizer, shards: shardMeta, tensors: tensors };
  return { manifest: manifest, shards: shards };
}

module.exports = { BRIK_VERSION: BRIK_VERSION, BRIK_ALIGN: BRIK_ALIGN, alignUp: alignUp, brikDataStart: brikDataStart,
  serializeBrik: serializeBrik, parseBrikHeader: parseBrikHeader, parseBrik: parseBrik,
  computeShardBases: computeShardBases, tensorBytes: tensorBytes, packShard: packShard, assembleBrik: assembleBrik };
