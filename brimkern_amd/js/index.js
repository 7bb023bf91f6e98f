'use strict';
// JavaScript host of the MI355X quantized matmul library: a drop-in for the quantized-matmul surface
// of the reference's WebGpuEngine (src/lib/webgpu/kernels.ts), over the N-API addon brik.node and
// through it the C ABI of include/brik.h. Node 12 compatible CommonJS (no ?. / ??).
//
//   reference (kernels.ts)                          here
//   uploadGpuRaw(bytes)                 :1032-1042  engine.uploadGpuRaw(bytes) -> DeviceBuffer
//   matmulQ4(a, nib, sc, mn, m, k, n)   :1046-1053  engine.matmulQ4(...)  -> Promise<Float32Array>
//   matmulQ4Tiled / matmulQ4Shared      :1055-1075  aliases of matmulQ4 (one entry picks the kernel by m)
//   matmulQ3(a, lo, hi, sc, mn, m, k, n):1080-1087  engine.matmulQ3(...)
//   matmulQ8(a, codes, sc, m, k, n)     :1140-1147  engine.matmulQ8(...), matmulQ8Tiled / Shared aliases
//   recMM(enc, trash, a, w, m, k, n)    :1562-1567  engine.recMM(trash, a, w, m, k, n) / mm(a, w, m, k, n[, out])
//                                                    (device resident, dispatch on the handle's shape:
//                                                    q3 / nib / codes; pooled output put on trash)
//   storage / release / releaseGpu /    :903-956,   engine.storage(bytes), release(bufs), releaseGpu(bufs),
//   trimPool / readGpu                  :1434-1458  trimPool(keep), readGpu(buf, n)
//   queue.writeBuffer                   :231-235    engine.writeBuffer(buf, data[, offset]) (no wait)
//   dequantGpuQ4/Q3/Q8 Q4W/Q3W/Q8W path  model.ts:214-270  engine.weightFromBlob(fmt, blob, nElems)
//   destroyWeight(b)                     model.ts:274-280  engine.destroyWeight(w)
//   decodeTopKQ8 head + sampling passes :1934-1968  engine.lmHeadTopK(x, w, d, vocab, recent, penalty, softcap, K)
//                                                    -> Promise<{ids: Uint32Array, vals: Float32Array}>
//   softcap_logits / penalize_logits /  :1940-1958  engine.logitsTopK(logits, vocab, recent, penalty, softcap, K)
//   top_k passes on a logits buffer                  (in place, like the reference's passes)
//   quantizeToBytes(type, data, n, dt)  :281-331    engine.quantizeToBytes(type, data, n, dtype[, chunk]) -> Promise<Uint8Array>
//   f32ToQ8Gpu / f32ToQ4Gpu             :986-1010   engine.quantize(dtype, src, n) -> device weight handle
//   matmulT(a, w, m, k, n, wF16=true)   :410-426    engine.matmulT(a, w, m, k, n, true) -> Promise<Float32Array>
//   (MATMUL_T_F16W, shaders.ts:2240)                 (w: f16 bits on the device); engine.mmF16(a, w, m, k, n[, out])
//   session conv2d with a q8 / q4 weight :1369-1374  engine.conv2d(inp, w, bias, Cin, H, W, Cout, kh, kw, st, pd[, out])
//   (recConv2dDirectQ8 / Q4)            :1233-1256  (device resident; inputs may be Float32Arrays)
//   .brik container (container.ts)                   require('./container'): parseBrik, serializeBrik, ...;
//                                                    engine.weightFromContainer(parsed, name)
//
// Plane arguments may be DeviceBuffers, plane views ({ptr: BigInt}) or BigInt addresses. Errors
// (bad shapes, K % 32 != 0, misalignment, no device) carry .code "BRIK_E...": the promise-returning
// methods (the readback ops, top-k, quantizeToBytes, matmulT, selfValidate) reject with them, the
// device-resident ones (mm, gemvPlan, conv2d, ...) throw; the reference validated nothing and let
// WebGPU fail silently. DeviceBuffers free their memory on destroy() or, if dropped, when collected.
//   selfValidate()                      :2255-2459  engine.selfValidate() -> Promise<boolean>, validationFailure

const path = require('path');
const planes = require('./planes');
const container = require('./container');

let native = null;
function loadNative() {
  if (native === null) native = require(path.join(__dirname, 'brik.node'));   // throws if not built
  return native;
}

const FMT = { q8: 8, q4: 4, q3: 3 };
const OPT_PATH = 1;
const OPT_GEMV_VARIANT = 2;

// A device allocation owned by this object: destroy() frees it at once; if the object is dropped
// without destroy(), the addon's finalizer frees it when the garbage collector reclaims the handle
// (the reference releases its buffers through destroy() or lets the GC take them, kernels.ts:903-956).

// The native job object of a plan job {x, w, y, K, N[, gate, norm, res, eps, onePlus, act]}.
function jobSpec(j) {
  const w = j.w;
  const s = { x: j.x, p0: w.nib || w.codes || w.lo, p1: w.hi || null, scales: w.sc, mins: w.mn || null,
    y: j.y, K: j.K, N: j.N };
  if (j.gate) s.gate = j.gate;
  if (j.norm) s.normW = j.norm;
  if (j.res) s.res = j.res;
  if (j.eps !== undefined) s.eps = j.eps;
  s.flags = (j.onePlus ? 1 : 0) | (j.act === 'gelu' ? 2 : 0);
  return s;
}

function planHandle(nat, plan) {
  return { run: function () { nat.gemvPlanRun(plan); }, destroy: function () { nat.gemvPlanDestroy(plan); } };
}
class DeviceBuffer {
  constructor(engine, handle, size) {
    this.engine = engine;
    this.handle = handle;                             // addon handle (owns the allocation)
    this.ptr = engine.native.bufferPtr(handle);       // BigInt device address
    this.size = size;                                 // bytes
  }
  // A plane view `offset` bytes into the buffer.
  view(offset) { return { ptr: this.ptr + BigInt(offset), buffer: this }; }
  destroy() {
    if (this.ptr !== null) {
      this.engine.native.freeBuffer(this.handle);
      this.ptr = null;
    }
  }
}

function einval(msg) {
  const e = new Error('BRIK_EINVAL: ' + msg);
  e.code = 'BRIK_EINVAL';
  return e;
}

function toBytes(data) {
  if (data instanceof Uint8Array) return data;
  if (ArrayBuffer.isView(data)) return new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
  if (data instanceof ArrayBuffer) return new Uint8Array(data);
  throw new TypeError('expected bytes (TypedArray / ArrayBuffer)');
}

class Engine {
  constructor(device) {
    this.native = loadNative();
    this.ctx = this.native.createContext(device === undefined ? 0 : device);
    // scratch pool by exact byte size, as the reference's storage() / release() (kernels.ts:903-956):
    // buffers return to it after use and are handed out again; stream order makes the reuse safe (a
    // call enqueued later runs after every earlier reader of the buffer)
    this._pool = new Map();
    this._pooled = new WeakSet();
  }

  static deviceCount() { return loadNative().deviceCount(); }

  // ---- memory ---------------------------------------------------------------------------------
  alloc(bytes) { return new DeviceBuffer(this, this.native.allocBuffer(this.ctx, Math.max(bytes, 1)), bytes); }

  // Device buffers allocated through this engine and not yet freed (by destroy() or the GC).
  liveBuffers() { return this.native.liveBuffers(this.ctx); }

  // Persistent device copy of raw bytes, padded to a 4-byte multiple (kernels.ts:1032-1042).
  uploadGpuRaw(bytes) {
    const b = toBytes(bytes);
    const size = Math.ceil(b.byteLength / 4) * 4;
    const buf = this.alloc(size);
    if (b.byteLength) this.native.h2d(this.ctx, buf.ptr, b);
    if (size !== b.byteLength) {
      const tail = new Uint8Array(size - b.byteLength);
      this.native.h2d(this.ctx, buf.ptr + BigInt(b.byteLength), tail);
    }
    return buf;
  }

  uploadGpu(f32) { return this.uploadGpuRaw(f32); }

  // ---- scratch pool (kernels.ts:903-956, 1418-1458) ----------------------------------------------
  // A device buffer of `bytes` from the pool (or a new one): the reference's storage().
  storage(bytes) {
    const free = this._pool.get(bytes);
    if (free && free.length) {
      const b = free.pop();
      this._pooled.delete(b);
      return b;
    }
    const b = this.alloc(bytes);
    b._poolSize = bytes;
    return b;
  }

  // Return buffers: pooled scratch (from storage) goes back to the pool, anything else is destroyed; a
  // buffer already in the pool is skipped (a double release would hand it out twice).
  release(buffers) {
    for (const b of buffers) {
      if (!b) continue;
      if (b._poolSize !== undefined) {
        if (this._pooled.has(b) || b.ptr === null) continue;
        this._pooled.add(b);
        let list = this._pool.get(b._poolSize);
        if (!list) { list = []; this._pool.set(b._poolSize, list); }
        list.push(b);
        continue;
      }
      if (typeof b.destroy === 'function') b.destroy();
    }
  }

  releaseGpu(buffers) { this.release(buffers); }

  // Shrink the pool to about keepBytes, largest buffers first (trimPool, kernels.ts:1440-1455).
  trimPool(keepBytes) {
    const keep = keepBytes === undefined ? 64 * 1024 * 1024 : keepBytes;
    let kept = 0;
    this._pool.forEach(function (list, size) { kept += size * list.length; });
    const sizes = Array.from(this._pool.keys()).sort(function (a, b) { return b - a; });
    for (const size of sizes) {
      const list = this._pool.get(size);
      while (list.length && kept > keep) {
        const b = list.pop();
        this._pooled.delete(b);
        b.destroy();
        kept -= size;
      }
    }
  }

  // Bytes held by the pool's free buffers.
  poolBytes() {
    let n = 0;
    this._pool.forEach(function (list, size) { n += size * list.length; });
    return n;
  }

  // Read nElems f32 of a device buffer back (readGpu, kernels.ts:1434).
  readGpu(buf, nElems) { return this.readBackAsync(buf, nElems * 4); }

  // Upload without waiting for earlier work (queue.writeBuffer, kernels.ts:231-235): the bytes are
  // staged at once, so `data` may be reused when this returns.
  writeBuffer(buf, data, offset) {
    const b = toBytes(data);
    const ptr = (typeof buf === 'bigint' ? buf : buf.ptr) + BigInt(offset || 0);
    if (b.byteLength) this.native.h2dAsync(this.ctx, ptr, b);
  }

  // ---- recorded launches ---------------------------------------------------------------------------
  // record(fn): the library calls fn() makes (plan runs, mm, ...) captured once into a HIP graph, not
  // run; the returned {launch(), destroy()} replays them, as the reference records a decode step into
  // one command encoder and submits it. Workspaces must already have their size (run fn() once before).
  record(fn) {
    const nat = this.native;
    nat.graphBegin(this.ctx);
    let g = null;
    try {
      fn();
    } finally {
      g = nat.graphEnd(this.ctx);
    }
    return { launch: function () { nat.graphLaunch(g); }, destroy: function () { nat.graphDestroy(g); } };
  }

  readBack(buf, bytes) {
    const ptr = typeof buf === 'bigint' ? buf : buf.ptr;
    return new Float32Array(this.native.d2h(this.ctx, ptr, bytes));
  }

  // Asynchronous form (readBack / mapAsync, kernels.ts:244-258): resolves once the work enqueued so far
  // has run, without blocking the JS thread meanwhile. The callback refers to `buf`, so a DeviceBuffer
  // stays reachable (its finalizer cannot free the memory) until the copy out of it has completed.
  readBackAsync(buf, bytes) {
    const ptr = typeof buf === 'bigint' ? buf : buf.ptr;
    return this.native.readbackAsync(this.ctx, ptr, bytes).then(function (ab) {
      void buf;   // a reference from the closure is what keeps the buffer alive
      return new Float32Array(ab);
    });
  }

  // A quantized weight handle from one packed .brik blob: one upload, planes addressed in place.
  // Shapes as model.ts:214-270 builds them: {nib, sc, mn} | {codes, sc} | {q3: true, lo, hi, sc, mn}.
  weightFromBlob(fmt, blob, nElems) {
    const offs = planes.planeOffsets(fmt, nElems);
    const b = toBytes(blob);
    const len = planes.byteLength(fmt, nElems);
    if (b.byteLength < len) throw new Error(fmt + ' blob of ' + b.byteLength + ' bytes is shorter than ' + len);
    const buf = this.uploadGpuRaw(b.subarray(0, len));
    const h = { _buf: buf };
    Object.keys(offs).forEach(function (k) { h[k] = buf.view(offs[k][0]); });
    if (fmt === 'q3') h.q3 = true;
    return h;
  }

  destroyWeight(w) {
    if (!w) return;
    if (w._buf) { w._buf.destroy(); return; }
    ['nib', 'codes', 'lo', 'hi', 'sc', 'mn'].forEach(function (k) {
      if (w[k] && typeof w[k].destroy === 'function') w[k].destroy();
    });
  }

  // ---- readback ops (reference signatures) -----------------------------------------------------
  // Upload a, enqueue the matmul and read y back without blocking the JS thread: the upload is staged
  // and enqueued without waiting for earlier work (writeBuffer), the readback resolves through a fence.
  // A bad argument or a library error rejects the promise. x and y come from the scratch pool and go
  // back to it once the readback has completed.
  async _readback(fn, a, planeArgs, m, k, n) {
    const x = a instanceof Float32Array ? a : Float32Array.from(a);
    if (x.length !== m * k) throw einval('activation has ' + x.length + ' floats, expected m*k = ' + m * k);
    const xb = this.storage(Math.max(x.byteLength, 4));
    const yb = this.storage(Math.max(m * n * 4, 4));
    try {
      this.writeBuffer(xb, x);
      fn.apply(this.native, [this.ctx, xb.ptr].concat(planeArgs, [yb.ptr, m, k, n]));
      return await this.readBackAsync(yb, m * n * 4);
    } finally {
      this.release([xb, yb]);
    }
  }

  matmulQ4(a, nib, sc, mn, m, k, n) { return this._readback(this.native.matmulQ4, a, [nib, sc, mn], m, k, n); }
  matmulQ4Tiled(a, nib, sc, mn, m, k, n) { return this.matmulQ4(a, nib, sc, mn, m, k, n); }
  matmulQ4Shared(a, nib, sc, mn, m, k, n) { return this.matmulQ4(a, nib, sc, mn, m, k, n); }

  matmulQ8(a, codes, sc, m, k, n) { return this._readback(this.native.matmulQ8, a, [codes, sc], m, k, n); }
  matmulQ8Tiled(a, codes, sc, m, k, n) { return this.matmulQ8(a, codes, sc, m, k, n); }
  matmulQ8Shared(a, codes, sc, m, k, n) { return this.matmulQ8(a, codes, sc, m, k, n); }

  matmulQ3(a, lo, hi, sc, mn, m, k, n) { return this._readback(this.native.matmulQ3, a, [lo, hi, sc, mn], m, k, n); }

  // The reference's load-time gate (selfValidate, kernels.ts:2255-2459): runs every quantized matmul
  // check of the library (brik_self_validate) and resolves true, or false with validationFailure set
  // to the failing check's name, as the reference does (useModelEngine.ts:243-249 refuses the model).
  async selfValidate() {
    this.validationFailure = null;
    const stage = this.native.selfValidate(this.ctx);
    if (stage === null) return true;
    this.validationFailure = stage;
    return false;
  }

  // ---- recorded (device-resident) form: recMM ---------------------------------------------------
  // recMM(trash, a, w, m, k, n) (kernels.ts:1521-1567): the output comes from the scratch pool and is
  // pushed onto `trash`; release(trash) returns it once the caller is done (the reference releases its
  // trash after the submit). mm(a, w, m, k, n[, out[, trash]]): into `out`, else a pooled buffer put
  // on `trash` if one is given, else a new buffer the caller owns.
  recMM(trash, a, w, m, k, n) { return this.mm(a, w, m, k, n, null, trash); }

  mm(a, w, m, k, n, out, trash) {
    let y = out;
    if (!y) {
      if (trash) {
        y = this.storage(Math.max(m * n * 4, 4));
        trash.push(y);
      } else {
        y = this.alloc(m * n * 4);
      }
    }
    if (w && w.q3) this.native.matmulQ3(this.ctx, a, w.lo, w.hi, w.sc, w.mn, y, m, k, n);
    else if (w && w.nib) this.native.matmulQ4(this.ctx, a, w.nib, w.sc, w.mn, y, m, k, n);
    else if (w && w.codes) this.native.matmulQ8(this.ctx, a, w.codes, w.sc, y, m, k, n);
    else {
      const e = new Error('BRIK_EINVAL: mm: weight handle is not a q3/q4/q8 handle');
      e.code = 'BRIK_EINVAL';
      throw e;
    }
    return y;
  }

  // Expert-grouped q4 matmul over a stacked [E, N, K] q4 weight (no reference counterpart).
  moeMatmulQ4(xSorted, rowOff, w, ySorted, E, R, K, N) {
    this.native.moeMatmulQ4(this.ctx, xSorted, rowOff, w.nib, w.sc, w.mn, ySorted, E, R, K, N);
    return ySorted;
  }

  // Two stacked [E, N, K] q4 weights on the same routed rows (an MoE layer's gate and up), one launch.
  moeMatmulQ4x2(xSorted, rowOff, wa, ya, wb, yb, E, R, K, N) {
    this.native.moeMatmulQ4x2(this.ctx, xSorted, rowOff, wa.nib, wa.sc, wa.mn, ya, wb.nib, wb.sc, wb.mn, yb, E, R, K, N);
    return [ya, yb];
  }

  // Grouped decode GEMV plan: jobs [{x, w, y, K, N}] (one format), executed by one launch per run().
  // Optional per job, the fusions of brik_gemv_job_ex (the ops recordLayerKV records around recMM,
  // kernels.ts:1701-1741): norm (RMSNorm gain buffer), eps, onePlus (Gemma 1 + w gain), gate (the
  // SwiGLU / GeGLU gate buffer, x being "up"), act ('gelu' for GeGLU), res (residual added to y).
  gemvPlan(fmt, jobs) {
    const nat = this.native;
    const plan = nat.gemvPlanCreate(this.ctx, FMT[fmt], jobs.map(jobSpec));
    return planHandle(nat, plan);
  }

  // The feed-forward half of a layer as linked plans (brik_gemv_plan_create_glu): gate and up jobs on
  // one input, then down on act(gate) * up (down.gate = gate.y, down.x = up.y; act: 'gelu' or SiLU).
  // Returns [gateUp, down]; run them in that order. Outputs equal those of two ordinary plans (within
  // f32 rounding for gate and up).
  gemvPlanGlu(fmt, gate, up, down) {
    const nat = this.native;
    const pair = nat.gemvPlanCreateGlu(this.ctx, FMT[fmt], jobSpec(gate), jobSpec(up), jobSpec(down));
    return [planHandle(nat, pair[0]), planHandle(nat, pair[1])];
  }

  // ---- sampling pre-work (decodeTopKQ8) --------------------------------------------------------
  async _topK(run, recent, K) {
    const ids = Array.from(new Set(recent || []));              // each id once, as the reference's callers do
    const rb = ids.length ? this.uploadGpuRaw(Int32Array.from(ids)) : null;
    const ob = this.alloc(8 * K);
    try {
      run(rb ? rb.ptr : null, ids.length, ob.ptr, ob.ptr + BigInt(4 * K));
      const raw = new Uint32Array(await this.native.readbackAsync(this.ctx, ob.ptr, 8 * K));
      return { ids: raw.slice(0, K), vals: new Float32Array(raw.buffer.slice(4 * K, 8 * K)) };
    } finally {
      ob.destroy();
      if (rb) rb.destroy();
    }
  }

  // softcap -> repetition penalty -> top-K on a device logits buffer (modified in place), kernels.ts:1940-1958.
  async logitsTopK(logits, vocab, recent, penalty, softcap, K) {
    const k = K === undefined ? 64 : K;
    const nat = this.native, ctx = this.ctx;
    return this._topK(function (rec, nrec, ids, vals) {
      nat.logitsTopK(ctx, logits, rec, ids, vals, vocab, nrec, k, penalty || 0, softcap || 0);
    }, recent, k);
  }

  // decodeTopKQ8's LM head and passes (kernels.ts:1934-1968) for one row x (Float32Array[d] or device
  // buffer): one launch for the whole vocab (no tiling), then the passes; K ids + values come back.
  async lmHeadTopK(x, w, d, vocab, recent, penalty, softcap, K) {
    const k = K === undefined ? 64 : K;
    const nat = this.native, ctx = this.ctx;
    const xb = (x instanceof Float32Array || Array.isArray(x)) ? this.uploadGpuRaw(Float32Array.from(x)) : null;
    const xp = xb ? xb.ptr : x;
    const fmt = w.q3 ? FMT.q3 : w.nib ? FMT.q4 : FMT.q8;
    try {
      return await this._topK(function (rec, nrec, ids, vals) {
        nat.lmHeadTopK(ctx, fmt, xp, w.nib || w.codes || w.lo, w.hi || null, w.sc, w.mn || null, rec, ids, vals,
          d, vocab, nrec, k, penalty || 0, softcap || 0);
      }, recent, k);
    } finally {
      if (xb) xb.destroy();
    }
  }

  dequant(fmt, w, out, nElems) {
    if (fmt === 'q8') this.native.dequantQ8(this.ctx, w.codes, w.sc, out, nElems);
    else if (fmt === 'q4') this.native.dequantQ4(this.ctx, w.nib, w.sc, w.mn, out, nElems);
    else this.native.dequantQ3(this.ctx, w.lo, w.hi, w.sc, w.mn, out, nElems);
    return out;
  }

  // ---- encoding (the conversion pipeline's GPU quantizer) ------------------------------------------
  // Tensor bytes -> packed .brik bytes (packQ8 / packQ4 / packQ3 layout), quantized on the GPU and
  // read back, like quantizeToBytes (kernels.ts:281-331). The bytes equal the CPU encoders'
  // (encodeTensor -> packQ*, codec.ts:17-29) for every input. `type` is the source encoding: 'F32',
  // 'F16' (decoded as kernels.ts:3213-3222 does), or a .brik quant 'Q8W' / 'Q4W' / 'Q3W' (dequantized
  // on the GPU first). `dtype`: 'q8' | 'q4' | 'q3'. The work runs in chunks of `chunkOverride`
  // elements (default 2^26), rounded to whole groups (whole 512-element blocks for quant sources),
  // so the device holds one chunk at a time; any chunking gives the same bytes.
  async quantizeToBytes(type, data, nElems, dtype, chunkOverride) {
    const src = toBytes(data);
    if (!FMT[dtype]) throw einval('quantizeToBytes: unknown dtype ' + dtype);
    if (!(nElems >= 0) || nElems % 32 !== 0) throw einval('quantizeToBytes: nElems ' + nElems + ' is not a multiple of 32');
    const quantSrc = { Q8W: 'q8', Q4W: 'q4', Q3W: 'q3' }[type];
    const need = type === 'F32' ? 4 * nElems : type === 'F16' ? 2 * nElems : quantSrc ? planes.byteLength(quantSrc, nElems) : -1;
    if (need < 0) throw einval('quantizeToBytes: unsupported source type ' + type);
    if (src.byteLength < need) throw einval('quantizeToBytes: ' + type + ' data has ' + src.byteLength + ' bytes, need ' + need);
    const out = new Uint8Array(planes.byteLength(dtype, nElems));
    if (nElems === 0) return out;
    const unit = quantSrc ? 512 : 32;
    let chunk = chunkOverride === undefined ? (1 << 26) : chunkOverride;
    chunk = Math.max(unit, Math.floor(chunk / unit) * unit);
    chunk = Math.min(chunk, nElems);
    const outOffs = planes.planeOffsets(dtype, nElems);
    const chunkOffs = planes.planeOffsets(dtype, Math.ceil(chunk / 32) * 32);
    const nat = this.native, ctx = this.ctx;
    const f32 = this.alloc(4 * chunk);
    const qbuf = this.alloc(planes.byteLength(dtype, Math.ceil(chunk / 32) * 32));
    const stage = type === 'F16' ? this.alloc(2 * chunk) : null;
    const w = quantSrc ? this.weightFromBlob(quantSrc, src, nElems) : null;
    // bytes per element of each plane (codes 1, nibbles 1/2, lo 1/4, hi 1/8, scales and mins 2/32)
    const perElem = { codes: 1, nib: 0.5, lo: 0.25, hi: 0.125, sc: 1 / 16, mn: 1 / 16 };
    try {
      for (let e0 = 0; e0 < nElems; e0 += chunk) {
        const ce = Math.min(chunk, nElems - e0);
        if (type === 'F32') {
          nat.h2d(ctx, f32.ptr, src.subarray(4 * e0, 4 * (e0 + ce)));
        } else if (type === 'F16') {
          nat.h2d(ctx, stage.ptr, src.subarray(2 * e0, 2 * (e0 + ce)));
          nat.f16ToF32(ctx, stage.ptr, f32.ptr, ce);
        } else {
          const at = function (p) { return w[p].ptr + BigInt(e0 * perElem[p]); };
          if (quantSrc === 'q8') nat.dequantQ8(ctx, at('codes'), at('sc'), f32.ptr, ce);
          else if (quantSrc === 'q4') nat.dequantQ4(ctx, at('nib'), at('sc'), at('mn'), f32.ptr, ce);
          else nat.dequantQ3(ctx, at('lo'), at('hi'), at('sc'), at('mn'), f32.ptr, ce);
        }
        const dst = function (p) { return qbuf.ptr + BigInt(chunkOffs[p][0]); };
        const names = Object.keys(outOffs);
        nat.quantize(ctx, FMT[dtype], f32.ptr, dst(names[0]), dtype === 'q3' ? dst('hi') : null, dst('sc'),
          dtype === 'q8' ? null : dst('mn'), ce);
        for (const p of names) {
          const len = ce * perElem[p];
          out.set(new Uint8Array(await nat.readbackAsync(ctx, dst(p), len)), outOffs[p][0] + e0 * perElem[p]);
        }
      }
    } finally {
      f32.destroy();
      qbuf.destroy();
      if (stage) stage.destroy();
      if (w) this.destroyWeight(w);
    }
    return out;
  }

  // f32ToQ8Gpu / f32ToQ4Gpu (kernels.ts:986-1010) and the q3 analogue: a device f32 buffer of nElems
  // values -> a device weight handle (one buffer in packQ* layout, planes addressed in place) that
  // mm / matmul* consume directly; the bytes are the CPU encoder's.
  quantize(dtype, src, nElems) {
    if (!FMT[dtype]) throw einval('quantize: unknown dtype ' + dtype);
    const offs = planes.planeOffsets(dtype, nElems);
    const buf = this.alloc(planes.byteLength(dtype, nElems));
    const h = { _buf: buf };
    Object.keys(offs).forEach(function (k) { h[k] = buf.view(offs[k][0]); });
    try {
      this.native.quantize(this.ctx, FMT[dtype], src, h.codes || h.nib || h.lo, h.hi || null, h.sc, h.mn || null, nElems);
    } catch (e) {
      buf.destroy();
      throw e;
    }
    if (dtype === 'q3') h.q3 = true;
    return h;
  }

  // matmulT with an f16 weight (kernels.ts:410-426 -> MATMUL_T_F16W): w is a device buffer / address of
  // N x K IEEE f16 values (uploadGpuRaw of the raw bytes). f32 weights (wF16 false) are outside this
  // library and throw BRIK_EINVAL.
  async matmulT(a, w, m, k, n, wF16) {
    if (!wF16) throw einval('matmulT: only f16 weights (wF16 = true) are handled here');
    return this._readback(this.native.matmulF16W, a, [w], m, k, n);
  }

  // Device-resident form of matmulT with an f16 weight.
  mmF16(a, w, m, k, n, out) {
    const y = out || this.alloc(m * n * 4);
    this.native.matmulF16W(this.ctx, a, w, y, m, k, n);
    return y;
  }

  // The recording session's conv2d for a quantized weight (kernels.ts:1369-1374, recConv2dDirectQ8 / Q4
  // at :1233-1256): w is a {codes, sc} or {nib, sc, mn} handle (f32 weights are outside this library);
  // inp and bias are device buffers or Float32Arrays (uploaded for the call). Returns the device
  // buffer out [Cout, OH, OW] (allocated when not given).
  conv2d(inp, w, bias, Cin, H, W, Cout, kh, kw, stride, pad, out) {
    const st = stride === undefined ? 1 : stride, pd = pad === undefined ? 0 : pad;
    const fmt = w && w.nib ? FMT.q4 : w && w.codes && !w.q3 ? FMT.q8 : 0;
    if (!fmt) throw einval('conv2d: the weight must be a q8 {codes, sc} or q4 {nib, sc, mn} handle');
    const OH = Math.floor((H + 2 * pd - kh) / st) + 1, OW = Math.floor((W + 2 * pd - kw) / st) + 1;
    const tmp = [];
    const dev = function (self, v) {
      if (v instanceof Float32Array) { const b = self.uploadGpu(v); tmp.push(b); return b.ptr; }
      return v;
    };
    const y = out || this.alloc(Math.max(Cout * OH * OW, 1) * 4);
    try {
      this.native.conv2d(this.ctx, fmt, dev(this, inp), w.nib || w.codes, w.sc, w.mn || null, dev(this, bias) || null,
        y, Cin, H, W, Cout, kh, kw, st, pd);
    } catch (e) {
      if (!out) y.destroy();
      throw e;
    } finally {
      tmp.forEach(function (b) { b.destroy(); });
    }
    return y;
  }

  // A weight handle for tensor `name` of a parsed .brik file (container.parseBrik): its packed bytes
  // uploaded once, planes addressed in place (weightFromBlob). Quantized dtypes only.
  weightFromContainer(parsed, name) {
    const t = container.tensorBytes(parsed, name);
    if (!FMT[t.entry.dtype]) throw einval('weightFromContainer: ' + name + ' has dtype ' + t.entry.dtype + ', not q8/q4/q3');
    return this.weightFromBlob(t.entry.dtype, t.bytes, t.entry.nElems);
  }

  setOption(key, value) { this.native.setOption(this.ctx, key, value); }
  sync() { this.native.sync(this.ctx); }
  timerBegin() { this.native.timerBegin(this.ctx); }
  timerEnd() { return this.native.timerEnd(this.ctx); }
}

module.exports = { Engine: Engine, DeviceBuffer: DeviceBuffer, planes: planes, container: container, FMT: FMT,
  OPT_PATH: OPT_PATH, OPT_GEMV_VARIANT: OPT_GEMV_VARIANT, loadNative: loadNative };
