'use strict';
// GPU checks of the JavaScript host's asynchronous surface and buffer lifetime (brimkern_amd/js over
// the N-API addon): readbacks resolve through stream fences off the JS thread, results of concurrent
// calls land in their own promises, bad arguments reject instead of throwing, dropped DeviceBuffers
// are freed by their finalizers (and keep their context alive until then), selfValidate passes; the
// scratch pool (storage / release / trimPool), recMM's pooled outputs, recorded launches, and readback
// ops that neither allocate per call nor wait for earlier work before returning.
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

  // 5. temporaries of the readback ops go back to the scratch pool: the live count is the base plus the
  // pool's free buffers, and trimming the pool returns it to the base
  {
    const pooled = engine.liveBuffers() - base;
    check('readback temporaries are pooled', pooled >= 2 && engine.poolBytes() > 0,
      { live: engine.liveBuffers(), base: base, poolBytes: engine.poolBytes() });
    engine.trimPool(0);
    check('trimPool(0) frees the pooled temporaries', engine.liveBuffers() === base && engine.poolBytes() === 0,
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

  // 8. the scratch pool (storage / release, kernels.ts:903-956): exact-size reuse, a double release
  // does not hand one buffer out twice, release destroys what is not pooled, trimPool frees
  {
    const a = engine.storage(4096);
    engine.release([a]);
    const b = engine.storage(4096);
    check('storage reuses a released buffer of the same size', a === b, {});
    engine.release([b, b]);
    const c1 = engine.storage(4096), c2 = engine.storage(4096);
    check('a double release is ignored', c1 !== c2 && c1 === b, {});
    const d = engine.storage(8192);
    check('another size is another buffer', d !== c1 && d !== c2, {});
    const own = engine.alloc(256);
    engine.release([c1, c2, d, own, null]);
    check('release destroys a buffer that is not pooled', own.ptr === null, {});
    check('the pool holds the released sizes', engine.poolBytes() === 2 * 4096 + 8192, { bytes: engine.poolBytes() });
    engine.trimPool(4096);
    check('trimPool drops the largest first down to keepBytes', engine.poolBytes() <= 4096, { bytes: engine.poolBytes() });
    engine.trimPool(0);
    check('trimPool(0) empties the pool', engine.poolBytes() === 0 && engine.liveBuffers() === base,
      { live: engine.liveBuffers(), base: base });
  }

  // 9. recMM(trash, ...): a pooled output on the trash, equal to the readback op; after release the next
  // call gets the same buffer, so a decode loop allocates nothing after its first step
  {
    const K = 2560, N = 1024;
    const w = await makeWeight(engine, 21, N, K);
    const xh = randn(rng(22), K);
    const x = engine.uploadGpu(xh);
    const ref = await engine.matmulQ4(xh, w.h.nib, w.h.sc, w.h.mn, 1, K, N);
    let trash = [];
    const y0 = engine.recMM(trash, x, w.h, 1, K, N);
    const got = await engine.readGpu(y0, N);
    check('recMM output is on the trash', trash.length === 1 && trash[0] === y0, {});
    check('recMM equals the readback op', normwise(got, ref) === 0, { rel: normwise(got, ref) });
    engine.release(trash);
    const live0 = engine.liveBuffers();
    let same = true;
    for (let i = 0; i < 100; i++) {
      trash = [];
      const y = engine.recMM(trash, x, w.h, 1, K, N);
      same = same && y === y0;
      engine.release(trash);
    }
    check('recMM reuses its pooled output across steps', same && engine.liveBuffers() === live0,
      { live: engine.liveBuffers(), live0: live0 });
    // the readback ops reuse their pooled temporaries the same way
    const live1 = engine.liveBuffers();
    for (let i = 0; i < 20; i++) await engine.matmulQ4(xh, w.h.nib, w.h.sc, w.h.mn, 1, K, N);
    check('readback ops allocate nothing per call', engine.liveBuffers() === live1,
      { live: engine.liveBuffers(), live1: live1 });
    x.destroy();
    engine.destroyWeight(w.h);
    engine.trimPool(0);
  }

  // 10. record(): launches captured once and replayed give the eager results (with the inputs changed
  // between replays: the graph keeps addresses, not contents)
  {
    const K = 1024, N = 768;
    const w = await makeWeight(engine, 23, N, K);
    const x = engine.alloc(4 * K), y = engine.alloc(4 * N);
    engine.writeBuffer(x, randn(rng(24), K));
    engine.mm(x, w.h, 1, K, N, y);                 // workspaces at size before the capture
    const g = engine.record(function () { engine.mm(x, w.h, 1, K, N, y); });
    let ok = true;
    for (let rep = 0; rep < 3; rep++) {
      const xh = randn(rng(30 + rep), K);
      engine.writeBuffer(x, xh);
      engine.writeBuffer(y, new Float32Array(N).fill(NaN));
      g.launch();
      const got = await engine.readGpu(y, N);
      const ref = await engine.matmulQ4(xh, w.h.nib, w.h.sc, w.h.mn, 1, K, N);
      ok = ok && normwise(got, ref) === 0;
    }
    g.destroy();
    check('recorded launches replay to the eager result', ok, {});
    [x, y].forEach(function (b) { b.destroy(); });
    engine.destroyWeight(w.h);
    engine.trimPool(0);
  }

  // 11. a readback op issued behind a long queue of work returns at once: the upload is staged and
  // enqueued without waiting (queue.writeBuffer), and the promise resolves after the queue drains
  {
    const K = 4096, N = 4096, M = 512;
    const big = await makeWeight(engine, 25, N, K);
    const xb = engine.uploadGpu(randn(rng(26), M * K));
    const yb = engine.alloc(M * N * 4);
    const w = await makeWeight(engine, 27, 512, 512);
    const xs = randn(rng(28), 512);
    await engine.matmulQ4(xs, w.h.nib, w.h.sc, w.h.mn, 1, 512, 512);   // pool and staging ring warm
    engine.mm(xb, big.h, M, K, N, yb);
    await engine.readGpu(yb, 4);
    const g = engine.record(function () { for (let i = 0; i < 100; i++) engine.mm(xb, big.h, M, K, N, yb); });
    for (let attempt = 0; attempt < 2; attempt++) {
      const t0 = process.hrtime.bigint();
      g.launch();
      g.launch();
      const t1 = process.hrtime.bigint();
      const p = engine.matmulQ4(xs, w.h.nib, w.h.sc, w.h.mn, 1, 512, 512);
      const t2 = process.hrtime.bigint();
      let ticks = 0, done = false;
      setImmediate(function spin() { if (!done) { ticks++; setImmediate(spin); } });
      const y = await p;
      done = true;
      const t3 = process.hrtime.bigint();
      const issue = Number(t2 - t1) / 1e6, total = Number(t3 - t0) / 1e6;
      const ref = cpuQ4(w.bytes, xs, 1, 512, 512);
      const rel = normwise(y, ref);
      if (attempt === 1 || (total > 4 && issue < 0.1 * total)) {
        check('matmulQ4 behind a long queue returns without waiting', total > 4 && issue < 0.1 * total,
          { issue_ms: issue, queue_ms: total });
        check('the event loop turns while it is pending', ticks >= 1, { ticks: ticks });
        check('its result is correct', rel <= 1e-5, { rel: rel });
        break;
      }
    }
    g.destroy();
    [xb, yb].forEach(function (b) { b.destroy(); });
    engine.destroyWeight(big.h);
    engine.destroyWeight(w.h);
    engine.trimPool(0);
  }

  const failed = results.filter(function (r) { return !r.ok; }).length;
  console.log(JSON.stringify({ checks: results.length, failed: failed }));
  process.exit(failed ? 1 : 0);
}

main().catch(function (e) { console.error(e && e.stack ? e.stack : e); process.exit(2); });
