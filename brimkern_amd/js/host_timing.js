'use strict';
// Host-side timing of the JavaScript engine (bench.py runs it under node and reports the line beside its
// own Python figures): what a Node host pays per call through the N-API addon, eager and replayed from a
// recorded graph, on the Qwen3-4B decode shapes with q4 weights.
//   mm: engine.mm at M = 1, K = 2560, N = 1024 (the k/v projection), rotating over weight copies that
//       exceed the 256 MB last-level cache;
//   layer: a decoder layer's matmul side as four fused plans (q/k/v, wo, the GLU pair, down) over 8
//          distinct layers, plan.run() per plan;
//   readback: an awaited engine.matmulQ4 (upload, kernel, fenced readback) on the k/v shape.
// The weights are random bytes of valid .brik q4 layout (timing only: values do not matter), scales and
// mins small finite f16. Prints one JSON line.
const path = require('path');
const brik = require(path.join(__dirname, 'index.js'));

function q4Blob(N, K, seed) {
  const n = N * K, g = n / 32;
  const b = new Uint8Array(n / 2 + 4 * g);
  let s = seed >>> 0;
  for (let i = 0; i < b.length; i += 4) {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    b[i] = s; b[i + 1] = s >>> 8; b[i + 2] = s >>> 16; b[i + 3] = s >>> 24;
  }
  const dv = new DataView(b.buffer);
  for (let j = 0; j < g; j++) {
    dv.setUint16(n / 2 + 2 * j, 0x2000 | (j & 0x3ff), true);          // scale ~ 0.008 .. 0.016
    dv.setUint16(n / 2 + 2 * g + 2 * j, 0xA400 | (j & 0x3ff), true);  // min ~ -0.016 .. -0.031
  }
  return b;
}

function usPer(t0, count) { return Number(process.hrtime.bigint() - t0) / 1e3 / count; }

async function main() {
  const e = new brik.Engine(0);
  const out = {};
  // mm on the k/v shape
  {
    const K = 2560, N = 1024, copies = 328;
    const blob = q4Blob(N, K, 1);
    const ws = [];
    for (let i = 0; i < copies; i++) ws.push(e.weightFromBlob('q4', blob, N * K));
    const x = e.uploadGpu(new Float32Array(K).fill(0.5));
    const y = e.alloc(4 * N);
    for (let i = 0; i < copies; i++) e.mm(x, ws[i], 1, K, N, y);
    e.sync();
    const calls = 4 * copies;
    let t0 = process.hrtime.bigint();
    for (let i = 0; i < calls; i++) e.mm(x, ws[i % copies], 1, K, N, y);
    const issue = usPer(t0, calls);
    e.sync();
    const wall = usPer(t0, calls);
    const g = e.record(function () { for (let i = 0; i < copies; i++) e.mm(x, ws[i], 1, K, N, y); });
    g.launch();
    e.sync();
    t0 = process.hrtime.bigint();
    for (let r = 0; r < 4; r++) g.launch();
    e.sync();
    const replay = usPer(t0, 4 * copies);
    g.destroy();
    // awaited readback round trips (one at a time), and 16 in flight
    const xh = new Float32Array(K).fill(0.25);
    const w0 = ws[0];
    await e.matmulQ4(xh, w0.nib, w0.sc, w0.mn, 1, K, N);
    t0 = process.hrtime.bigint();
    for (let i = 0; i < 200; i++) await e.matmulQ4(xh, ws[i % copies].nib, ws[i % copies].sc, ws[i % copies].mn, 1, K, N);
    const rt = usPer(t0, 200);
    t0 = process.hrtime.bigint();
    for (let b = 0; b < 25; b++) {
      const ps = [];
      for (let i = 0; i < 16; i++) ps.push(e.matmulQ4(xh, ws[i].nib, ws[i].sc, ws[i].mn, 1, K, N));
      await Promise.all(ps);
    }
    const rt16 = usPer(t0, 400);
    out.mm_kv_K2560_N1024 = { issue_us: +issue.toFixed(2), wall_us: +wall.toFixed(2), replay_us: +replay.toFixed(2),
      copies: copies, note: 'issue: JS loop of mm calls until the last returns; wall: until the stream drains; ' +
        'replay: the same calls recorded once (engine.record) and replayed' };
    out.readback_matmulQ4_kv = { awaited_us: +rt.toFixed(1), sixteen_in_flight_us: +rt16.toFixed(1),
      note: 'engine.matmulQ4(Float32Array) -> Promise<Float32Array>: staged upload, kernel, fenced readback' };
    ws.forEach(function (w) { e.destroyWeight(w); });
    [x, y].forEach(function (b) { b.destroy(); });
    e.trimPool(0);
  }
  // a decoder layer as four fused plans, 8 distinct layers
  {
    const d = 2560, qd = 4096, kvd = 1024, ffn = 9728, L = 8;
    const shapes = { q: [d, qd], k: [d, kvd], v: [d, kvd], o: [qd, d], gate: [d, ffn], up: [d, ffn], down: [ffn, d] };
    const blobs = {};
    Object.keys(shapes).forEach(function (n, i) { blobs[n] = q4Blob(shapes[n][1], shapes[n][0], 10 + i); });
    const buf = function (n, v) { return e.uploadGpu(new Float32Array(n).fill(v)); };
    const h = buf(d, 0.1), attn = buf(qd, 0.1), norm = buf(d, 1.0);
    const q = e.alloc(4 * qd), k = e.alloc(4 * kvd), v = e.alloc(4 * kvd), gt = e.alloc(4 * ffn), up = e.alloc(4 * ffn);
    const plans = [], weights = [];
    for (let l = 0; l < L; l++) {
      const w = {};
      Object.keys(shapes).forEach(function (n) { w[n] = e.weightFromBlob('q4', blobs[n], shapes[n][0] * shapes[n][1]); });
      weights.push(w);
      plans.push(e.gemvPlan('q4', [{ x: h, norm: norm, eps: 1e-6, w: w.q, y: q, K: d, N: qd },
        { x: h, norm: norm, eps: 1e-6, w: w.k, y: k, K: d, N: kvd }, { x: h, norm: norm, eps: 1e-6, w: w.v, y: v, K: d, N: kvd }]));
      plans.push(e.gemvPlan('q4', [{ x: attn, w: w.o, y: h, res: h, K: qd, N: d }]));
      const glu = e.gemvPlanGlu('q4', { x: h, norm: norm, eps: 1e-6, w: w.gate, y: gt, K: d, N: ffn },
        { x: h, norm: norm, eps: 1e-6, w: w.up, y: up, K: d, N: ffn }, { x: up, gate: gt, w: w.down, y: h, res: h, K: ffn, N: d });
      plans.push(glu[0], glu[1]);
    }
    const step = function () { for (const p of plans) p.run(); };
    step();
    e.sync();
    const reps = 50;
    let t0 = process.hrtime.bigint();
    for (let r = 0; r < reps; r++) step();
    const issue = usPer(t0, reps * L);
    e.sync();
    const wall = usPer(t0, reps * L);
    const g = e.record(step);
    g.launch();
    e.sync();
    t0 = process.hrtime.bigint();
    for (let r = 0; r < reps; r++) g.launch();
    e.sync();
    const replay = usPer(t0, reps * L);
    g.destroy();
    out.layer_fused_plans_qwen3_4b = { issue_us_per_layer: +issue.toFixed(2), wall_us_per_layer: +wall.toFixed(2),
      replay_us_per_layer: +replay.toFixed(2), layers: L, launches_per_layer: 4,
      note: 'plan.run() x 4 per layer from JS; replay: the same runs recorded once and replayed' };
    plans.forEach(function (p) { p.destroy(); });
    weights.forEach(function (w) { Object.keys(w).forEach(function (n) { e.destroyWeight(w[n]); }); });
  }
  out.node = process.version;
  console.log(JSON.stringify(out));
}

main().catch(function (err) { console.error(err && err.stack ? err.stack : err); process.exit(1); });
