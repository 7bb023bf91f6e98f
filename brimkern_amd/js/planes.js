'use strict';
// .brik quantized tensor layouts: byte lengths and plane offsets inside one packed blob.
//
// Same offsets as the reference's unpackQ8 / unpackQ4 / unpackQ3 (src/lib/brik/q8web.ts:65-72,
// q4web.ts:70-80, q3web.ts:80-95) and lengths as q8ByteLength / q4ByteLength / q3ByteLength
// (q8web.ts:23-26, q4web.ts:23-26, q3web.ts:29-32). Node 12 compatible CommonJS.

const GROUP = 32;

function checkN(fmt, n) {
  if (n % GROUP !== 0) throw new Error(fmt + ': nElems ' + n + ' is not a multiple of ' + GROUP);
}

function q8ByteLength(n) { return n + (n / GROUP) * 2; }
function q4ByteLength(n) { return n / 2 + (n / GROUP) * 4; }
function q3ByteLength(n) { return (n / 16) * 4 + (n / 32) * 4 + (n / GROUP) * 4; }

function byteLength(fmt, n) {
  checkN(fmt, n);
  if (fmt === 'q8') return q8ByteLength(n);
  if (fmt === 'q4') return q4ByteLength(n);
  if (fmt === 'q3') return q3ByteLength(n);
  throw new Error('unknown format ' + fmt);
}

// {plane: [byteOffset, byteLength]} for an n-element tensor.
function planeOffsets(fmt, n) {
  checkN(fmt, n);
  const g = n / GROUP;
  if (fmt === 'q8') return { codes: [0, n], sc: [n, 2 * g] };
  if (fmt === 'q4') return { nib: [0, n / 2], sc: [n / 2, 2 * g], mn: [n / 2 + 2 * g, 2 * g] };
  if (fmt === 'q3') {
    const lb = (n / 16) * 4, hb = (n / 32) * 4;
    return { lo: [0, lb], hi: [lb, hb], sc: [lb + hb, 2 * g], mn: [lb + hb + 2 * g, 2 * g] };
  }
  throw new Error('unknown format ' + fmt);
}

module.exports = { GROUP: GROUP, q8ByteLength: q8ByteLength, q4ByteLength: q4ByteLength,
  q3ByteLength: q3ByteLength, byteLength: byteLength, planeOffsets: planeOffsets };
