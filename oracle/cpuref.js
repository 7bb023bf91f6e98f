'use strict';
// JavaScript restatement of the reference's CPU matmul (TEST INFRASTRUCTURE ONLY — a checker and
// the timed CPU baseline, never the product path).
//
// Follows, in the reference's own language and numeric model:
//   f16BitsToF32 ........ src/lib/brik/f16.ts:25-34
//   dequantizeQ8/Q4/Q3 .. src/lib/brik/q8web.ts:74-83, q4web.ts:82-96, q3web.ts:97-110
//   reference matmul .... src/lib/webgpu/kernels.ts:2335-2337 (Wd = dequantize(q) into a
//                         Float32Array; ref[c] = sum over i of a[i] * Wd[c*k + i] in a JS double)
//   f32ToF16Bits ........ src/lib/brik/f16.ts:8-22
//   quantizeQ8/Q4/Q3 .... src/lib/brik/q8web.ts:28-50, q4web.ts:28-53, q3web.ts:34-60, packed as
//                         packQ8/Q4/Q3 (q8web.ts:55-62, q4web.ts:58-66, q3web.ts:65-76)
// Node 12 compatible (CommonJS, no optional chaining / nullish coalescing).
//
// CLI (used by bench.py's cpu_baseline leg and the encoder tests):
//   node oracle/cpuref.js <fmt> <M> <K> <N> <input.bin> <output.bin> [reps]
//   node oracle/cpuref.js quantize <dtype> <input.f32> <output.bin> [reps]   (packed bytes of the f32 input)
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

function f32ToF16Bits(val) {
  const f = new Float32Array(1);
  const i = new Uint32Array(f.buffer);
  f[0] = val;
  const x = i[0];
  const sign = (x >> 16) & 0x8000;
  let exp = ((x >> 23) & 0xff) - 127 + 15;
  let mant = x & 0x7fffff;
  if (exp <= 0) return sign;
  if (exp >= 31) return sign | 0x7bff;
  mant = (mant >> 13) + ((mant >> 12) & 1);
  if (mant === 0x400) { mant = 0; exp += 1; }
  return sign | (exp << 10) | (mant & 0x3ff);
}

// The encoders, in the reference's numeric model (JS doubles, Math.round, typed-array stores), each
// returning the packed bytes. levels = 127 (q8, symmetric) / 15 (q4) / 7 (q3).
function quantize(dtype, data) {
  const n = data.length;
  if (n % GROUP !== 0) throw new Error(dtype + ': length ' + n + ' not a multiple of ' + GROUP);
  const groups = n / GROUP;
  const scales = new Uint16Array(groups), mins = new Uint16Array(groups);
  const codes = new Int8Array(dtype === 'q8' ? n : 0);
  const nibbles = new Uint8Array(dtype === 'q4' ? n / 2 : 0);
  const lo = new Uint32Array(dtype === 'q3' ? n / 16 : 0), hi = new Uint32Array(dtype === 'q3' ? n / 32 : 0);
  for (let g = 0; g < groups; g++) {
    const base = g * GROUP;
    if (dtype === 'q8') {
      let amax = 0;
      for (let i = 0; i < GROUP; i++) { const a = Math.abs(data[base + i]); if (a > amax) amax = a; }
      const sH = f32ToF16Bits(amax / 127 || 1e-8);
      scales[g] = sH;
      const s = f16BitsToF32(sH) || 1e-8;
      for (let i = 0; i < GROUP; i++) {
        let q = Math.round(data[base + i] / s);
        q = q < -127 ? -127 : q > 127 ? 127 : q;
        codes[base + i] = q;
      }
      continue;
    }
    const L = dtype === 'q4' ? 15 : 7;
    let mn = Infinity, mx = -Infinity;
    for (let i = 0; i < GROUP; i++) { const v = data[base + i]; if (v < mn) mn = v; if (v > mx) mx = v; }
    const sH = f32ToF16Bits((mx - mn) / L || 1e-8), mH = f32ToF16Bits(mn);
    scales[g] = sH; mins[g] = mH;
    const s = f16BitsToF32(sH) || 1e-8, m = f16BitsToF32(mH);
    for (let i = 0; i < GROUP; i++) {
      let q = Math.round((data[base + i] - m) / s);
      q = q < 0 ? 0 : q > L ? L : q;
      const idx = base + i;
      if (dtype === 'q4') {
        if ((i & 1) === 0) nibbles[idx >> 1] = q;
        else nibbles[idx >> 1] |= q << 4;
      } else {
        lo[idx >> 4] |= (q & 3) << ((idx & 15) * 2);
        hi[idx >> 5] |= (q >> 2) << (idx & 31);
      }
    }
  }
  const parts = dtype === 'q8' ? [codes, scales] : dtype === 'q4' ? [nibbles, scales, mins] : [lo, hi, scales, mins];
  const len = parts.reduce(function (a, p) { return a + p.byteLength; }, 0);
  const out = new Uint8Array(len);
  let off = 0;
  parts.forEach(function (p) {
    out.set(new Uint8Array(p.buffer, p.byteOffset, p.byteLength), off);
    off += p.byteLength;
  });
  return out;
}

module.exports = { f16BitsToF32: f16BitsToF32, f32ToF16Bits: f32ToF16Bits, planes: planes, dequantize: dequantize,
  matmulRef: matmulRef, cpuMatmul: cpuMatmul, quantize: quantize };

function quantizeCli(argv) {
  const fs = require('fs');
  const buf = fs.readFileSync(argv[2]);
  const data = new Float32Array(buf.buffer.slice(buf.byteOffset, buf.byteOffset + (buf.byteLength & ~3)));
  const reps = argv.length > 4 ? +argv[4] : 1;
  let best = Infinity, total = 0, out = null;
  for (let r = 0; r < reps; r++) {
    const t0 = process.hrtime();
    out = quantize(argv[1], data);
    const d = process.hrtime(t0);
    const ms = d[0] * 1e3 + d[1] / 1e6;
    best = Math.min(best, ms);
    total += ms;
  }
  fs.writeFileSync(argv[3], Buffer.from(out.buffer, out.byteOffset, out.byteLength));
  process.stdout.write(JSON.stringify({ ms: best, total_ms: total, reps: reps, dtype: argv[1], n: data.length }) + '\n');
}

if (require.main === module && process.argv[2] === 'quantize') {
  quantizeCli(process.argv.slice(2));
} else if (require.main === module) {
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
