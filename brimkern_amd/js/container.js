'use strict';
// The single-file .brik container: reader, writer and the shard layout of a converted model, with the
// file bytes of the reference's writer (src/lib/brik/container.ts, codec.ts:62-98, convert.ts:37-89,
// loader.ts:57-66, format.ts:6-8) so that a file made on either side loads on the other.
//
//   bytes [0, 4)        "BRIK"
//         [4, 8)        format version, u32 little-endian (1)
//         [8, 12)       L = manifest length in bytes, u32 little-endian
//         [12, 12 + L)  manifest, JSON.stringify of the manifest object, UTF-8
//         [D, end)      data section, D = 12 + L rounded up to 16: the shards back to back by id
//
// Inside a shard every tensor starts on a 16-byte boundary and the shard's length is a multiple of 16,
// so every tensor of the file is 16-byte aligned. A tensor lives at D + base(shard) + offset.
//
// The module is built on one placement routine (`place`) used at both levels: tensors inside a shard
// (16-byte runs) and shards inside the data section (runs already 16-byte multiples). Error messages
// are the reference's, word for word, so callers that match on them see the same errors. Values are
// not encoded here: quantized tensors arrive as packed planes (engine.quantizeToBytes).

const BRIK_VERSION = 1;
const BRIK_ALIGN = 16;
const MAGIC = [0x42, 0x52, 0x49, 0x4b];   // "BRIK"
const FIXED = 12;                          // magic + version + manifest length

function alignUp(n, align) {
  const a = align === undefined ? BRIK_ALIGN : align;
  return Math.ceil(n / a) * a;
}

function brikDataStart(manifestByteLength) { return alignUp(FIXED + manifestByteLength); }

function asBytes(data) {
  if (data instanceof Uint8Array) return data;
  if (ArrayBuffer.isView(data)) return new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
  if (data instanceof ArrayBuffer) return new Uint8Array(data);
  throw new TypeError('expected bytes (TypedArray / ArrayBuffer)');
}

// Runs of the given lengths laid end to end, each starting on a multiple of `align`: their start
// offsets and the end of the last one.
function place(lengths, align) {
  const at = new Array(lengths.length);
  let end = 0;
  for (let i = 0; i < lengths.length; i++) {
    at[i] = alignUp(end, align);
    end = at[i] + lengths[i];
  }
  return { at: at, end: end };
}

function byId(shards) { return shards.slice().sort(function (a, b) { return a.id - b.id; }); }

// ---- reading --------------------------------------------------------------------------------------

// The fixed header and the manifest, from the leading bytes of a file (parseBrikHeader, container.ts:71-81).
function parseBrikHeader(data) {
  const b = asBytes(data);
  if (b.length < FIXED) throw new Error('BRIK: fichier tronqué (en-tête)');
  const seal = String.fromCharCode(b[0], b[1], b[2], b[3]);
  if (MAGIC.some(function (c, i) { return b[i] !== c; })) throw new Error('BRIK: sceau magique absent (' + seal + ')');
  const dv = new DataView(b.buffer, b.byteOffset, FIXED);
  const length = dv.getUint32(8, true);
  if (length > b.length - FIXED) throw new Error('BRIK: manifeste tronqué');
  const json = Buffer.from(b.buffer, b.byteOffset + FIXED, length).toString('utf8');
  return { manifest: JSON.parse(json), version: dv.getUint32(4, true), dataStart: brikDataStart(length) };
}

// The header plus `data`, a view of the data section (parseBrik, container.ts:84-87).
function parseBrik(data) {
  const b = asBytes(data);
  const h = parseBrikHeader(b);
  h.data = b.subarray(h.dataStart);
  return h;
}

// Byte offset of each shard in the data section, indexed by shard id (loader.ts:57-66).
function computeShardBases(shards) {
  const ordered = byId(shards);
  const p = place(ordered.map(function (s) { return s.byteLength; }), 1);
  const bases = [];
  ordered.forEach(function (s, i) { bases[s.id] = p.at[i]; });
  return bases;
}

// One tensor of a parsed file: its manifest entry and a view of its bytes (no copy).
function tensorBytes(parsed, name) {
  const entry = parsed.manifest.tensors[name];
  if (!entry) throw new Error('BRIK: tenseur absent : ' + name);
  const base = computeShardBases(parsed.manifest.shards)[entry.shard];
  const from = base + entry.offset, to = from + entry.byteLength;
  if (base === undefined || to > parsed.data.length) throw new Error('BRIK: tenseur tronqué : ' + name);
  return { entry: entry, bytes: parsed.data.subarray(from, to) };
}

// ---- writing --------------------------------------------------------------------------------------

// The file bytes for a manifest and its shards [{file, bytes}] (serializeBrik, container.ts:30-58):
// every shard the manifest lists must be supplied at the length it declares.
function serializeBrik(manifest, shards) {
  const supplied = {};
  shards.forEach(function (s) { supplied[s.file] = asBytes(s.bytes); });
  const table = byId(manifest.shards).map(function (s) {
    const bytes = Object.prototype.hasOwnProperty.call(supplied, s.file) ? supplied[s.file] : null;
    if (!bytes) throw new Error('shard manquant : ' + s.file);
    if (bytes.length !== s.byteLength) {
      throw new Error('taille de shard incohérente pour ' + s.file + ' : ' + bytes.length + ' ≠ ' + s.byteLength);
    }
    return bytes;
  });
  const json = Buffer.from(JSON.stringify(manifest), 'utf8');
  const start = brikDataStart(json.length);
  const section = place(table.map(function (b) { return b.length; }), 1);
  const file = new Uint8Array(start + section.end);
  file.set(MAGIC, 0);
  const dv = new DataView(file.buffer);
  dv.setUint32(4, BRIK_VERSION, true);
  dv.setUint32(8, json.length, true);
  file.set(json, FIXED);
  table.forEach(function (b, i) { file.set(b, start + section.at[i]); });
  return file;
}

function elementCount(t) {
  if (t.nElems !== undefined) return t.nElems;
  if (t.data) return t.data.length;
  let n = 1;
  for (const d of t.shape) n *= d;
  return n;
}

// Tensors [{name, dtype, shape, bytes | data (f32 only), nElems}] placed into one shard on 16-byte
// boundaries, the shard padded to 16 (packShard, codec.ts:62-98): {buffer, entries by name}.
function packShard(tensors, shardId) {
  const payloads = tensors.map(function (t) {
    if (t.bytes) return asBytes(t.bytes);
    if (t.dtype !== 'f32' || !t.data) throw new Error('packShard: ' + t.name + ' needs pre-encoded bytes for dtype ' + t.dtype);
    return asBytes(Float32Array.from(t.data));
  });
  const p = place(payloads.map(function (b) { return b.length; }), BRIK_ALIGN);
  const buffer = new Uint8Array(alignUp(p.end));
  const entries = {};
  tensors.forEach(function (t, i) {
    buffer.set(payloads[i], p.at[i]);
    entries[t.name] = { dtype: t.dtype, shape: t.shape, nElems: elementCount(t), shard: shardId, offset: p.at[i],
      byteLength: payloads[i].length };
  });
  return { buffer: buffer, entries: entries };
}

// Shard grouping of a converted model (convert.ts:37-89): the tensors of transformer block i
// ("blk.<i>.") form shard "layer-<i, 4 digits>", all others the "shared" shard; shard ids follow
// "shared" first, then the group names in string order; shard files are "shard-<id, 4 digits>.brik".
const BLOCK = /^blk\.(\d+)\./;
function groupOf(name) {
  const m = BLOCK.exec(name);
  return m ? 'layer-' + m[1].padStart(4, '0') : 'shared';
}
function groupRank(a, b) {
  if (a === b) return 0;
  if (a === 'shared') return -1;
  if (b === 'shared') return 1;
  return a.localeCompare(b);
}

// {model, arch, chat, tokenizer, tensors} -> {manifest, shards: [{file, bytes}]} (assembleBrik)
function assembleBrik(input) {
  const groups = {};
  input.tensors.forEach(function (t) {
    const g = groupOf(t.name);
    (groups[g] || (groups[g] = [])).push(t);
  });
  const manifest = { format: 'brik', version: BRIK_VERSION, model: input.model, arch: input.arch, chat: input.chat,
    tokenizer: input.tokenizer, shards: [], tensors: {} };
  const shards = Object.keys(groups).sort(groupRank).map(function (g, id) {
    const packed = packShard(groups[g], id);
    const file = 'shard-' + String(id).padStart(4, '0') + '.brik';
    Object.keys(packed.entries).forEach(function (n) { manifest.tensors[n] = packed.entries[n]; });
    manifest.shards.push({ id: id, file: file, byteLength: packed.buffer.length });
    return { file: file, bytes: packed.buffer };
  });
  return { manifest: manifest, shards: shards };
}

module.exports = { BRIK_VERSION: BRIK_VERSION, BRIK_ALIGN: BRIK_ALIGN, alignUp: alignUp, brikDataStart: brikDataStart,
  serializeBrik: serializeBrik, parseBrikHeader: parseBrikHeader, parseBrik: parseBrik,
  computeShardBases: computeShardBases, tensorBytes: tensorBytes, packShard: packShard, assembleBrik: assembleBrik };
