'use strict';
// GPU checks of the JavaScript host's asynchronous surface and buffer lifetime (brimkern_amd/js over
// the N-API addon): readbacks resolve through stream fences off the JS thread, results of concurrent
// calls land in their own promises, bad arguments reject instead of throwing, dropped DeviceBuffers
// are freed by their finalizers (and keep their context alive until then), and selfValidate passes.
// Run with --expose-gc; prints one JSON line, exit code 0 iff every check passed.
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

function rng(seed) {   // mulberry32
  let a = seed >>> 0;
  return function () {
    a = (a + 0x6D2B79F5) >>> 0;
    let t = a;
    t = Math.imul(t ^ (t >>> 15), t | 1);
    t ^= t + Math.imul(t ^ (t >>> 7), t | 61);
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
}

function randn(r, n) {
  const out = new Float32Array(n);
  for (let i = 0; i < n; i++) out[i] = (r() + r() + r() + r() - 2) * 1.7;
  return out;
}

function tick() { return new Promise(function (res) { setImmediate(res); }); }

async function collect() {
  for (let i = 0; i < 4; i++) { global.gc(); await tick(); }
}

// a q4 weight made by the device encoder from a seeded f32 matrix, plus its host bytes for cpuref
async function makeWeight(engine, seed, N, K) {
  const w = randn(rng(seed), N * K);
  const bytes = await engine.quantizeToBytes('F32', new Uint8Array(w.buffer), N * K, 'q4');
  return { bytes: bytes, h: engine.weightFromBlob('q4', bytes, N * K) };
}

function cpuQ4(bytes, x, M, K, N) { return cpuref.cpuMatmul('q4', x, bytes, M, K, N); }

async function main() {
  if (typeof global.gc !== 'function') throw new Error('run with node --expose-gc');
  const engine = new brik.Engine(0);
  const base = engine.liveBuffers();

  // 1. selfValidate: every load-time check of the quantized kernels passes
  {
    const ok = await engine.selfValidate();
    check('selfValidate resolves true', ok === true && engine.validationFailure === null,
      { ok: ok, failure: engine.validationFailure });
  }

  // 2. concurrent readbacks: each promise carries its own call's result
  {
    const K = 512, N = 384;
    const w = await makeWeight(engine, 11, N, K);
    const shapes = [1, 3, 8, 40, 130];
    const xs = shapes.map(function (m, i) { return randn(rng(100 + i), m * K); });
    const ps = shapes.map(function (m, i) { return engine.matmulQ4(xs[i], w.h.nib, w.h.sc, w.h.mn, m, K, N); });
    check('matmulQ4 returns a promise', ps.every(function (p) { return p instanceof Promise; }), {});
    const ys = await Promise.all(ps);
    shapes.forEach(function (m, i) {
      const r = cpuQ4(w.bytes, xs[i], m, K, N);
      const rel = normwise(ys[i], r);
      check('concurrent matmulQ4 m=' + m, ys[i].length === m * N && rel <= 1e-3, { rel: rel });
    });
    engine.destroyWeight(w.h);
  }

  // 3. the JS thread runs while a readback is pending: setImmediate callbacks fire before it resolves
  {
    const K = 4096, N = 4096, M = 512;
    const w = await makeWeight(engine, 12, N, K);
    const x = engine.uploadGpu(randn(rng(13), M * K));
    const y = engine.alloc(M * N * 4);
    for (let i = 0; i < 20; i++) engine.mm(x, w.h, M, K, N, y);
    let ticks = 0, done = false;
    const p = engine.readBackAsync(y, 4 * N).then(function (v) { done = true; return v; });
    setImmediate(function spin() { if (!done) { ticks++; setImmediate(spin); } });   // counts loop turns only
    const first = await p;
    check('event loop ran during a pending readback', ticks >= 1 && first.length === N, { ticks: ticks });
    [x, y].forEach(function (b) { b.destroy(); });
    engine.destroyWeight(w.h);
  }

  // 4. bad arguments reject the promise (no synchronous throw)
  {
    const K = 64, N = 64;
    const w = await makeWeight(engine, 14, N, K);
    let threw = false, p = null;
    try { p = engine.matmulQ4(new Float32Array(48), w.h.nib, w.h.sc, w.h.mn, 1, 48, N); } catch (e) { threw = true; }
    let code = null;
    if (p) { try { await p; } catch (e) { code = e.code; } }
    check('K % 32 != 0 rejects with BRIK_EINVAL', !threw && code === 'BRIK_EINVAL', { threw: threw, code: code });
    threw = false; p = null; code = null;
    try { p = engine.matmulQ4(new Float32Array(10), w.h.nib, w.h.sc, w.h.mn, 1, K, N); } catch (e) { threw = true; }
    if (p) { try { await p; } catch (e) { code = e.code; } }
    check('short activation rejects with BRIK_EINVAL', !threw && code === 'BRIK_EINVAL', { threw: threw, code: code });
    threw = false; p = null; code = null;
    try { p = engine.quantizeToBytes('F32', new Uint8Array(40), 10, 'q4'); } catch (e) { threw = true; }
    if (p) { try { await p; } catch (e) { code = e.code || e.name; } }
    check('quantizeToBytes of a ragged length rejects', !threw && code === 'BRIK_EINVAL', { threw: threw, code: code });
    // the engine still works after the rejections
    const x = randn(rng(15), 2 * K);
    const y = await engine.matmulQ4(x, w.h.nib, w.h.sc, w.h.mn, 2, K, N);
    const rel = normwise(y, cpuQ4(w.bytes, x, 2, K, N));
    check('rejected calls leave the engine usable', rel <= 1e-3, { rel: rel });
    engine.destroyWeight(w.h);
  }

  // 5. temporaries of the readback ops are freed: the live count returns to where it was
  {
    check('readback ops free their temporaries', engine.liveBuffers() === base,
      { live: engine.liveBuffers(), base: base });
  }

  // 6. dropped DeviceBuffers are freed by their finalizers
  {
    (function () { for (let i = 0; i < 64; i++) engine.alloc(1 << 16); })();
    const mid = engine.liveBuffers();
    await collect();
    const after = engine.liveBuffers();
    check('dropped buffers counted while live', mid >= base + 1, { mid: mid, base: base });
    check('finalizers free dropped buffers', after === base, { after: after, base: base });
    const b = engine.alloc(256);
    b.destroy();
    b.destroy();
    check('destroy() frees at once and twice is harmless', engine.liveBuffers() === base, { live: engine.liveBuffers() });
  }

  // 7. a buffer outlives its dropped engine: its handle keeps the context alive until it is collected
  {
    let handle = null, nat = null, ptr0 = null;
    (function () {
      const e2 = new brik.Engine(0);
      const b = e2.uploadGpu(Float32Array.from([1, 2, 3, 4]));
      handle = b.handle;
      nat = e2.native;
      ptr0 = b.ptr;
    })();
    await collect();           // the engine, its context handle and the DeviceBuffer wrapper are gone
    let err = null;
    try {
      if (nat.bufferPtr(handle) !== ptr0) err = 'address changed';
      nat.freeBuffer(handle);  // frees into the context the handle kept alive
    } catch (e) { err = e.message; }
    handle = null;
    await collect();           // the last reference goes: the context is destroyed here
    check('buffer outlives its dropped engine', err === null, { err: err });
  }

  const failed = results.filter(function (r) { return !r.ok; }).length;
  console.log(JSON.stringify({ checks: results.length, failed: failed }));
  process.exit(failed ? 1 : 0);
}

main().catch(function (e) { console.error(e && e.stack ? e.stack : e); process.exit(2); });
