'use strict';
// JavaScript restatement of the reference's CPU matmul (TEST INFRASTRUCTURE ONLY — a checker and
// the timed CPU baseline, never the product path).
//
// Follows, in the reference's own language and numeric model:
//   f16BitsToF32 ........ src/lib/brik/f16.ts:25-34
//   dequantizeQ8/Q4/Q3 .. src/lib/brik/q8web.ts:108-117, q4web.ts:199-213, q3web.ts:310-323
//   reference matmul .... src/lib/webgpu/kernels.ts:2335-2337 (Wd = dequantize(q) into a
//                         Float32Array; ref[c] = sum over i of a[i] * Wd[c*k + i] in a JS double)
// Node 12 compatible (CommonJS, no optional chaining / nullish coalescing).
//
// CLI (used by bench.py's cpu_baseline leg):
//   node oracle/cpuref.js <fmt> <M> <K> <N> <input.bin> <output.bin> [reps]
// input.bin = x (M*K f32) followed by the packed .brik blob of W [N, K]; output.bin receives y.
// Prints one JSON line: {"ms": best wall time of one full matmul incl. dequant, "total_ms": wall time
// of all reps, "reps": ...}.

const GROUP = 32;

function f16BitsToF32(h) {
  const s = (h >> 15) & 1;
  const e = (h >> 10) & 0x1f;
  const m = h & 0x3ff;
  let val;
  if (e === 0) val = m * 5.9604645e-8;
  else if (e === 31) val = m ? NaN : Infinity;
  else val = (1 + m / 1024) * Math.pow(2, e - 15);
  return s === 1 ? -val : val;
}

function planes(fmt, bytes, n) {
  const g = n / GROUP;
  const dv = new DataView(bytes.buffer, bytes.byteOffset, bytes.byteLength);
  const u16 = function (off, cnt) {
    const a = new Uint16Array(cnt);
    for (let i = 0; i < cnt; i++) a[i] = dv.getUint16(off + 2 * i, true);
    return a;
  };
  const u32 = function (off, cnt) {
    const a = new Uint32Array(cnt);
    for (let i = 0; i < cnt; i++) a[i] = dv.getUint32(off + 4 * i, true);
    return a;
  };
  if (fmt === 'q8') {
    return { codes: new Int8Array(bytes.buffer, bytes.byteOffset, n), scales: u16(n, g) };
  }
  if (fmt === 'q4') {
    const nl = n / 2;
    return { nibbles: bytes.subarray(0, nl), scales: u16(nl, g), mins: u16(nl + 2 * g, g) };
  }
  const lb = (n / 16) * 4, hb = (n / 32) * 4;
  return { lo: u32(0, n / 16), hi: u32(lb, n / 32), scales: u16(lb + hb, g), mins: u16(lb + hb + 2 * g, g) };
}

function dequantize(fmt, t, n) {
  const out = new Float32Array(n);
  const groups = n / GROUP;
  for (let g = 0; g < groups; g++) {
    const s = f16BitsToF32(t.scales[g]);
    const m = fmt === 'q8' ? 0 : f16BitsToF32(t.mins[g]);
    const base = g * GROUP;
    for (let i = 0; i < GROUP; i++) {
      const idx = base + i;
      if (fmt === 'q8') {
        out[idx] = t.codes[idx] * s;
      } else if (fmt === 'q4') {
        const byte = t.nibbles[idx >> 1];
        const q = (i & 1) === 0 ? (byte & 0xf) : (byte >> 4);
        out[idx] = q * s + m;
      } else {
        const q = ((t.lo[idx >> 4] >> ((idx & 15) * 2)) & 3) | (((t.hi[idx >> 5] >> (idx & 31)) & 1) << 2);
        out[idx] = q * s + m;
      }
    }
  }
  return out;
}

// kernels.ts:2335-2337 / 2364-2365: f64 running sum, one rounding into the Float32Array.
function matmulRef(a, Wd, m, k, n) {
  const ref = new Float32Array(m * n);
  for (let r = 0; r < m; r++) {
    for (let c = 0; c < n; c++) {
      let s = 0;
      for (let i = 0; i < k; i++) s += a[r * k + i] * Wd[c * k + i];
      ref[r * n + c] = s;
    }
  }
  return ref;
}

function cpuMatmul(fmt, a, blob, m, k, n) {
  const Wd = dequantize(fmt, planes(fmt, blob, n * k), n * k);
  return matmulRef(a, Wd, m, k, n);
}

module.exports = { f16BitsToF32: f16BitsToF32, planes: planes, dequantize: dequantize,
  matmulRef: matmulRef, cpuMatmul: cpuMatmul };

if (require.main === module) {
  const fs = require('fs');
  const argv = process.argv.slice(2);
  const fmt = argv[0], M = +argv[1], K = +argv[2], N = +argv[3];
  const reps = argv.length > 6 ? +argv[6] : 1;
  const buf = fs.readFileSync(argv[4]);
  const bytes = new Uint8Array(buf.buffer, buf.byteOffset, buf.byteLength);
  const a = new Float32Array(bytes.buffer.slice(bytes.byteOffset, bytes.byteOffset + M * K * 4));
  const blob = bytes.slice(M * K * 4);
  let best = Infinity, total = 0, y = null;
  for (let r = 0; r < reps; r++) {
    const t0 = process.hrtime();
    y = cpuMatmul(fmt, a, blob, M, K, N);
    const d = process.hrtime(t0);
    const ms = d[0] * 1e3 + d[1] / 1e6;
    best = Math.min(best, ms);
    total += ms;
  }
  fs.writeFileSync(argv[5], Buffer.from(y.buffer));
  process.stdout.write(JSON.stringify({ ms: best, total_ms: total, reps: reps, fmt: fmt, M: M, K: K, N: N }) + '\n');
}
