'use strict';
// GPU parity of the JavaScript host (brimkern_amd/js over the N-API addon) against the golden fixtures
// and against the JavaScript restatement of the reference CPU matmul (oracle/cpuref.js) on seeded
// inputs. Prints one JSON line; exit code 0 iff every check passed. Run by tests/test_js_host.py.
const fs = require('fs');
const path = require('path');
const root = path.join(__dirname, '..', '..');
const brik = require(path.join(root, 'brimkern_amd', 'js'));
const cpuref = require(path.join(root, 'oracle', 'cpuref.js'));

const results = [];
function check(name, ok, detail) {
  results.push({ name: name, ok: !!ok, detail: detail });
  if (!ok) console.error('FAIL ' + name + ' ' + JSON.stringify(detail));
}

function normwise(y, r) {
  let num = 0, den = 0;
  for (let i = 0; i < r.length; i++) {
    num = Math.max(num, Math.abs(y[i] - r[i]));
    den = Math.max(den, Math.abs(r[i]));
  }
  return den === 0 ? num : num / den;
}

// mulberry32: a small seeded generator for the JS-side inputs.
function rng(seed) {
  let a = seed >>> 0;
  return function () {
    a = (a + 0x6D2B79F5) >>> 0;
    let t = a;
    t = Math.imul(t ^ (t >>> 15), t | 1);
    t ^= t + Math.imul(t ^ (t >>> 7), t | 61);
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
}

function f16bits(v) {   // f32 -> f16 for normal-range positive/negative scales (test data only)
  const f = new Float32Array([v]);
  const x = new Uint32Array(f.buffer)[0];
  const sign = (x >>> 16) & 0x8000;
  let exp = ((x >>> 23) & 0xff) - 127 + 15;
  let mant = x & 0x7fffff;
  let r = (mant >>> 13) + ((mant >>> 12) & 1);
  if (r === 0x400) { r = 0; exp += 1; }
  return sign | (exp << 10) | (r & 0x3ff);
}

// kernels.ts:2836 ranking (stable sort) and :2862-2866 acceptance rule
function topkRule(got, ref, K) {
  const order = Array.from(ref.keys()).sort(function (a, b) { return ref[b] - ref[a]; }).slice(0, K);
  for (let r = 0; r < K; r++) {
    const okV = Math.abs(got.vals[r] - ref[order[r]]) <= 1e-4 * (1 + Math.abs(ref[order[r]]));
    const okI = Math.abs(ref[got.ids[r]] - got.vals[r]) <= 1e-4 * (1 + Math.abs(got.vals[r]));
    if (!okV || !okI) return false;
  }
  return got.ids.length === K && got.vals.length === K;
}

async function main() {
  const meta = JSON.parse(fs.readFileSync(path.join(root, 'tests', 'golden', 'golden.json')));
  const raw = fs.readFileSync(path.join(root, 'tests', 'golden', 'golden.bin'));
  const bytes = function (span) { return new Uint8Array(raw.buffer, raw.byteOffset + span[0], span[1]); };
  const f32 = function (span) { return new Float32Array(bytes(span).slice().buffer); };
  const engine = new brik.Engine(0);

  // 1. golden fixtures through the reference-shaped readback ops + dequant bit-exactness
  for (const c of meta.cases) {
    const n = c.N * c.K;
    const w = engine.weightFromBlob(c.fmt, bytes(c.blob), n);
    const x = f32(c.x);
    let y;
    if (c.fmt === 'q4') y = await engine.matmulQ4(x, w.nib, w.sc, w.mn, c.M, c.K, c.N);
    else if (c.fmt === 'q8') y = await engine.matmulQ8(x, w.codes, w.sc, c.M, c.K, c.N);
    else y = await engine.matmulQ3(x, w.lo, w.hi, w.sc, w.mn, c.M, c.K, c.N);
    const rel = normwise(y, f32(c.y));
    check('golden ' + c.name, rel <= (c.M === 1 ? 1e-5 : 1e-3), { rel: rel });
    const out = engine.alloc(n * 4);
    engine.dequant(c.fmt, w, out.ptr, n);
    const deq = new Uint32Array(engine.readBack(out, n * 4).buffer);
    const ref = new Uint32Array(f32(c.deq).buffer);
    let same = deq.length === ref.length;
    for (let i = 0; same && i < ref.length; i++) same = deq[i] === ref[i];
    check('dequant ' + c.name, same, {});
    out.destroy();
    engine.destroyWeight(w);
  }

  // 2. seeded q4 at a Qwen3-4B shape, GPU vs the JS CPU reference (oracle/cpuref.js)
  {
    const K = 2560, N = 1024, n = N * K;
    const r = rng(12345);
    const blob = new Uint8Array(brik.planes.byteLength('q4', n));
    for (let i = 0; i < n / 2; i++) blob[i] = (r() * 256) | 0;
    const dv = new DataView(blob.buffer);
    for (let g = 0; g < n / 32; g++) {
      const s = 0.005 + 0.015 * r();
      dv.setUint16(n / 2 + 2 * g, f16bits(s), true);
      dv.setUint16(n / 2 + n / 16 + 2 * g, f16bits(-7.5 * s), true);
    }
    const x = new Float32Array(K);
    for (let i = 0; i < K; i++) x[i] = 2 * r() - 1;
    const w = engine.weightFromBlob('q4', blob, n);
    const y = await engine.matmulQ4(x, w.nib, w.sc, w.mn, 1, K, N);
    const t0 = process.hrtime();
    const ref = cpuref.cpuMatmul('q4', x, blob, 1, K, N);
    const dt = process.hrtime(t0);
    check('q4 K2560 N1024 vs JS CPU reference', normwise(y, ref) <= 1e-5, { rel: normwise(y, ref), cpu_ms: dt[0] * 1e3 + dt[1] / 1e6 });

    // 3. recMM form: device-resident activation and output, dispatch on the handle shape
    const xb = engine.uploadGpu(x);
    const yb = engine.mm(xb.view(0), w, 1, K, N);
    check('mm (recMM) q4', normwise(engine.readBack(yb, N * 4), ref) <= 1e-5, {});

    // 4. grouped plan of two jobs sharing x
    const y2 = engine.alloc(N * 4), y3 = engine.alloc(N * 4);
    const plan = engine.gemvPlan('q4', [{ x: xb, w: w, y: y2, K: K, N: N }, { x: xb, w: w, y: y3, K: K, N: N }]);
    plan.run();
    check('gemv plan q4', normwise(engine.readBack(y2, N * 4), ref) <= 1e-5 &&
      normwise(engine.readBack(y3, N * 4), ref) <= 1e-5, {});
    plan.destroy();

    // 5. errors surface as exceptions with BRIK_* codes
    let code = null;
    try { await engine.matmulQ4(x.subarray(0, 48), w.nib, w.sc, w.mn, 1, 48, N); } catch (e) { code = e.code; }
    check('K % 32 != 0 throws BRIK_EINVAL', code === 'BRIK_EINVAL', { code: code });
    code = null;
    try { engine.mm(xb.view(4), w, 1, K, N, y2); } catch (e) { code = e.code; }
    check('misaligned activation throws BRIK_EALIGN', code === 'BRIK_EALIGN', { code: code });
    code = null;
    try { engine.mm(xb, {}, 1, K, N, y2); } catch (e) { code = e.code; }
    check('non-quantized handle throws BRIK_EINVAL', code === 'BRIK_EINVAL', { code: code });
    // 6. LM head + sampling pre-work over this weight as a 1024-token head (decodeTopKQ8's passes)
    const recent = [3, 500, 1023, 77];
    const cap = 20, pen = 1.3, TK = 32;
    const lref = Float32Array.from(ref, function (v) { return cap * Math.tanh(v / cap); });
    recent.forEach(function (id) { lref[id] = lref[id] > 0 ? lref[id] / pen : lref[id] * pen; });
    const got = await engine.lmHeadTopK(x, w, K, N, recent, pen, cap, TK);
    check('lmHeadTopK q4', topkRule(got, lref, TK), {});
    [xb, yb, y2, y3].forEach(function (b) { b.destroy(); });
    engine.destroyWeight(w);
  }

  // 7. the reference's own top_k validation (kernels.ts:2828-2870): vocab 152064, K 64, penalty 1.15,
  //    cap 30, logits U(-8, 8), 40 recent ids deduplicated, same CPU reference and acceptance rule
  {
    const vocab = 152064, TK = 64, penalty = 1.15, cap = 30;
    const r = rng(777);
    const logits = Float32Array.from({ length: vocab }, function () { return (r() * 2 - 1) * 8; });
    const recent = Array.from(new Set(Array.from({ length: 40 }, function () { return Math.floor(r() * vocab); })));
    const cpu = logits.slice();
    for (let i = 0; i < vocab; i++) cpu[i] = cap * Math.tanh(cpu[i] / cap);
    for (const id of recent) cpu[id] = cpu[id] > 0 ? cpu[id] / penalty : cpu[id] * penalty;
    const lb = engine.uploadGpuRaw(logits);
    const got = await engine.logitsTopK(lb, vocab, recent, penalty, cap, TK);
    check('logitsTopK reference validation case', topkRule(got, cpu, TK), {});
    lb.destroy();
  }

  // 8. the GPU encoder against the reference's CPU encoder (encodeTensor -> packQ*, restated in
  //    oracle/cpuref.js): quantizeToBytes in one pass and in chunks of 256 (kernels.ts:2461-2472),
  //    then a .brik file of the encoded tensors read back into a weight handle for the matmul
  {
    const r = rng(4242);
    const n = 32 * 51;
    const w = Float32Array.from({ length: n }, function () { return (r() * 2 - 1) * 3; });
    w[7] = NaN; w[40] = Infinity;
    for (let i = 64; i < 96; i++) w[i] = 0;
    for (let i = 96; i < 128; i++) w[i] = (i - 111.5) / 16;      // exact ties
    const bytes = new Uint8Array(w.buffer);
    for (const dt of ['q8', 'q4', 'q3']) {
      const cpu = cpuref.quantize(dt, w);
      const one = await engine.quantizeToBytes('F32', bytes, n, dt);
      const many = await engine.quantizeToBytes('F32', bytes, n, dt, 256);
      const same = function (a, b) { return a.length === b.length && a.every(function (v, i) { return v === b[i]; }); };
      check('quantizeToBytes ' + dt + ' equals the CPU encoder', same(one, cpu), {});
      check('quantizeToBytes ' + dt + ' chunked equals one pass', same(one, many), {});
    }
    const K = 256, N = 96;
    const wm = Float32Array.from({ length: N * K }, function () { return r() * 2 - 1; });
    const q4 = await engine.quantizeToBytes('F32', new Uint8Array(wm.buffer), N * K, 'q4');
    const c = brik.container;
    const built = c.assembleBrik({ model: { name: 't' }, arch: { d: K }, chat: { template: '', stopTokenIds: [] },
      tokenizer: { kind: 'hf-hub', id: 'x' },
      tensors: [{ name: 'blk.0.ffn_up.weight', dtype: 'q4', shape: [N, K], bytes: q4, nElems: N * K }] });
    const parsed = c.parseBrik(c.serializeBrik(built.manifest, built.shards));
    const hw = engine.weightFromContainer(parsed, 'blk.0.ffn_up.weight');
    const xv = Float32Array.from({ length: K }, function () { return r() * 2 - 1; });
    const y = await engine.matmulQ4(xv, hw.nib, hw.sc, hw.mn, 1, K, N);
    const ref = cpuref.cpuMatmul('q4', xv, q4, 1, K, N);
    check('weightFromContainer q4 -> matmulQ4', normwise(y, ref) <= 1e-5, { rel: normwise(y, ref) });
    engine.destroyWeight(hw);
    // device-resident encode (f32ToQ4Gpu analogue) feeding recMM
    const wb = engine.uploadGpu(wm);
    const hq = engine.quantize('q4', wb, N * K);
    const raw = new Uint8Array(engine.native.d2h(engine.ctx, hq._buf.ptr, q4.length));
    check('quantize (device handle) bytes', raw.every(function (v, i) { return v === q4[i]; }), {});
    const xb = engine.uploadGpu(xv);
    const yb = engine.mm(xb, hq, 1, K, N);
    check('quantize handle -> mm', normwise(engine.readBack(yb, N * 4), ref) <= 1e-5, {});
    [wb, xb, yb].forEach(function (b) { b.destroy(); });
    engine.destroyWeight(hq);
  }

  // 9. the session conv2d with quantized weights on the reference's validation shape (kernels.ts:3085-3120):
  //    Cin 8, 4x4, Cout 4, 3x3, stride 1, pad 1, against the reference loop (kernels.ts:3049-3061) on the
  //    dequantized weights
  {
    const r = rng(99);
    const Cin = 8, Hh = 4, Ww = 4, Cout = 4, kk = 3;
    const cx = Float32Array.from({ length: Cin * Hh * Ww }, function () { return r() * 2 - 1; });
    const cw = Float32Array.from({ length: Cout * Cin * kk * kk }, function () { return r() * 2 - 1; });
    const cb = Float32Array.from({ length: Cout }, function () { return r() * 2 - 1; });
    for (const dt of ['q8', 'q4']) {
      const blob = cpuref.quantize(dt, cw);
      const wd = cpuref.dequantize(dt, cpuref.planes(dt, blob, cw.length), cw.length);
      const ref = new Float32Array(Cout * Hh * Ww);
      for (let co = 0; co < Cout; co++)
        for (let oy = 0; oy < Hh; oy++)
          for (let ox = 0; ox < Ww; ox++) {
            let acc = cb[co];
            for (let ci = 0; ci < Cin; ci++)
              for (let ky = 0; ky < kk; ky++)
                for (let kx = 0; kx < kk; kx++) {
                  const iy = oy + ky - 1, ix = ox + kx - 1;
                  if (iy >= 0 && iy < Hh && ix >= 0 && ix < Ww)
                    acc += cx[ci * Hh * Ww + iy * Ww + ix] * wd[((co * Cin + ci) * kk + ky) * kk + kx];
                }
            ref[(co * Hh + oy) * Ww + ox] = acc;
          }
      const hw = engine.weightFromBlob(dt, blob, cw.length);
      const yb = engine.conv2d(cx, hw, cb, Cin, Hh, Ww, Cout, kk, kk, 1, 1);
      check('conv2d ' + dt + ' (session form)', normwise(engine.readBack(yb, ref.length * 4), ref) <= 1e-5, {});
      yb.destroy();
      engine.destroyWeight(hw);
    }
  }

  // 10. matmulT with an f16 weight (MATMUL_T_F16W): decode row and a small prefill, against the JS sum
  {
    const r = rng(1234);
    const K = 512, N = 96;
    const wf = Float32Array.from({ length: N * K }, function () { return (r() * 2 - 1) * 0.1; });
    const bits = new Uint16Array(N * K);
    for (let i = 0; i < bits.length; i++) bits[i] = cpuref.f32ToF16Bits(wf[i]);
    const wd = Float32Array.from(bits, function (h) { return cpuref.f16BitsToF32(h); });
    const wb = engine.uploadGpuRaw(bits);
    for (const m of [1, 4]) {
      const xv = Float32Array.from({ length: m * K }, function () { return r() * 2 - 1; });
      const y = await engine.matmulT(xv, wb, m, K, N, true);
      const ref = cpuref.matmulRef(xv, wd, m, K, N);
      check('matmulT f16 weight m=' + m, normwise(y, ref) <= (m === 1 ? 1e-5 : 1e-3), { rel: normwise(y, ref) });
    }
    let code = null;
    try { await engine.matmulT(new Float32Array(K), wb, 1, K, N, false); } catch (e) { code = e.code; }
    check('matmulT with f32 weights throws BRIK_EINVAL', code === 'BRIK_EINVAL', { code: code });
    wb.destroy();
  }

  // 11. expert-grouped q4 (moeMatmulQ4 / moeMatmulQ4x2): per-expert rows against the JS sum over the
  // dequantized expert slice; the two-tensor call equals two single calls bit for bit
  {
    const r = rng(4321);
    const E = 3, K = 128, N = 40, rowOff = [0, 5, 5, 12], R = 12;
    const mk = async function () {
      const wm = Float32Array.from({ length: E * N * K }, function () { return r() * 2 - 1; });
      const bytes = await engine.quantizeToBytes('F32', new Uint8Array(wm.buffer), E * N * K, 'q4');
      return { bytes: bytes, h: engine.weightFromBlob('q4', bytes, E * N * K) };
    };
    const wa = await mk(), wb = await mk();
    const xv = Float32Array.from({ length: R * K }, function () { return r() * 2 - 1; });
    const xb = engine.uploadGpu(xv), rb = engine.uploadGpuRaw(Int32Array.from(rowOff));
    const ys = [0, 1, 2, 3].map(function () { return engine.alloc(R * N * 4); });
    engine.moeMatmulQ4(xb, rb, wa.h, ys[0], E, R, K, N);
    engine.moeMatmulQ4(xb, rb, wb.h, ys[1], E, R, K, N);
    engine.moeMatmulQ4x2(xb, rb, wa.h, ys[2], wb.h, ys[3], E, R, K, N);
    const got = [];
    for (const y of ys) got.push(await engine.readBackAsync(y, R * N * 4));
    const same = function (a, b) { return a.every(function (v, i) { return Object.is(v, b[i]); }); };
    check('moeMatmulQ4x2 equals two moeMatmulQ4 calls', same(got[0], got[2]) && same(got[1], got[3]), {});
    [[wa, got[0]], [wb, got[1]]].forEach(function (pair, t) {
      const wd = cpuref.dequantize('q4', cpuref.planes('q4', pair[0].bytes, E * N * K), E * N * K);
      let worst = 0;
      for (let e = 0; e < E; e++) {
        const m = rowOff[e + 1] - rowOff[e];
        if (!m) continue;
        const ref = cpuref.matmulRef(xv.subarray(rowOff[e] * K, rowOff[e + 1] * K), wd.subarray(e * N * K, (e + 1) * N * K), m, K, N);
        worst = Math.max(worst, normwise(pair[1].subarray(rowOff[e] * N, rowOff[e + 1] * N), ref));
      }
      check('moeMatmulQ4 tensor ' + t + ' vs JS per-expert sum', worst <= 1e-3, { rel: worst });
    });
    [xb, rb].concat(ys).forEach(function (b) { b.destroy(); });
    engine.destroyWeight(wa.h);
    engine.destroyWeight(wb.h);
  }

  const failed = results.filter(function (r) { return !r.ok; }).length;
  process.stdout.write(JSON.stringify({ checks: results.length, failed: failed }) + '\n');
  process.exit(failed === 0 ? 0 : 1);
}

main().catch(function (e) { console.error(e && e.stack ? e.stack : e); process.exit(2); });
