// Device runtime for the attention operator on MI355X: the part of the WebGPU runtime
// (app/gpu/device.js) that the operator and its callers use, over the N-API addon
// (lib/supra_attn.node) and the C ABI behind it (include/supra_attn.h).
//
// - Tensor (app/gpu/device.js:41-55): a pooled device buffer plus a shape; release() returns the
//   buffer to the pool at once. That is safe because all work runs in order on one HIP stream: a
//   later kernel that reuses the buffer is ordered after every earlier kernel that read it.
// - GPU.empty / fromArray / upload / read / sync (app/gpu/device.js:144-191, 255-259).
// - Errors: a failed call throws synchronously, with err.code set to the C ABI status
//   ("SA_ERR_INVALID", "SA_ERR_UNSUPPORTED", "SA_ERR_HIP", "SA_ERR_ALIAS").
// - Device lost (app/gpu/device.js:134, 208): the first SA_ERR_HIP (the HIP runtime failed: a fault,
//   a reset, a lost device) is latched in gpu.lost, and every later operator call, read or sync
//   throws it again instead of issuing more work.
// - Profiler (app/gpu/device.js:272-325): GPU.create({ profile: true }) times every operator call
//   with a HIP event pair on the device stream; gpu.profiler.report() aggregates ms and flops by
//   operator name.
//
// Written for Node >= 12 (CommonJS, no optional chaining / nullish coalescing).
"use strict";

var path = require("path");

var ADDON_PATH = path.join(__dirname, "..", "lib", "supra_attn.node");

function loadNative() {
  return require(ADDON_PATH);
}

var ELEMENT_BYTES = { f32: 4, i32: 4, u8: 1 };

function product(shape) {
  var n = 1;
  for (var i = 0; i < shape.length; i++) n *= shape[i];
  return n;
}

function dtypeOf(arr) {
  if (arr instanceof Float32Array) return "f32";
  if (arr instanceof Int32Array) return "i32";
  if (arr instanceof Uint8Array) return "u8";
  throw new TypeError("fromArray takes a Float32Array, Int32Array or Uint8Array");
}

// Pooled device buffers, bucketed by rounded size: quarter-power-of-two steps above 1 KiB.
function BufferPool(native) {
  this.native = native;
  this.free = new Map();
  this.allocated = 0;
  this.peak = 0;
}

BufferPool.round = function (bytes) {
  var b = Math.max(256, bytes);
  if (b <= 1024) return Math.ceil(b / 256) * 256;
  var step = Math.pow(2, Math.floor(Math.log2(b))) / 4;
  return Math.ceil(b / step) * step;
};

BufferPool.prototype.get = function (bytes) {
  var size = BufferPool.round(bytes);
  var list = this.free.get(size);
  if (list && list.length) return { buf: list.pop(), size: size };
  var buf = this.native.malloc(size);
  this.allocated += size;
  this.peak = Math.max(this.peak, this.allocated);
  return { buf: buf, size: size };
};

BufferPool.prototype.put = function (buf, size) {
  if (!this.free.has(size)) this.free.set(size, []);
  this.free.get(size).push(buf);
};

BufferPool.prototype.trim = function () {
  var self = this;
  this.free.forEach(function (list, size) {
    for (var i = 0; i < list.length; i++) {
      self.native.free(list[i]);
      self.allocated -= size;
    }
  });
  this.free.clear();
};

function Tensor(gpu, buf, shape, bytes, dtype) {
  this.gpu = gpu;
  this.buf = buf;
  this.shape = shape;
  this.bytes = bytes;
  this.dtype = dtype || "f32";
}

Object.defineProperty(Tensor.prototype, "size", {
  get: function () {
    return product(this.shape);
  },
});

Tensor.prototype.release = function () {
  if (this.buf) this.gpu.pool.put(this.buf, this.bytes);
  this.buf = null;
};

// Per-operator timings aggregated by name (app/gpu/device.js:272-325). begin/end record a HIP event
// pair on the device stream around one operator's launches; collect() waits for the recorded pairs
// and folds them into { name, count, ms, flops } entries. Events are recycled.
function Profiler(native, capacity) {
  this.native = native;
  this.capacity = capacity || 2048;
  this.spare = [];
  this.pending = [];
  this.stats = new Map();
}

Profiler.prototype.event = function () {
  return this.spare.length ? this.spare.pop() : this.native.eventCreate();
};

Profiler.prototype.begin = function (meta) {
  var start = this.event();
  try {
    this.native.eventRecord(start);
  } catch (e) {
    this.spare.push(start);
    throw e;
  }
  return { meta: meta || { name: "?", flops: 0 }, start: start, stop: null };
};

Profiler.prototype.end = function (tok) {
  tok.stop = this.event();
  this.native.eventRecord(tok.stop);
  this.pending.push(tok);
  if (this.pending.length >= this.capacity) this.collect();
};

// An operator that threw launched nothing: its start event goes back unused.
Profiler.prototype.cancel = function (tok) {
  this.spare.push(tok.start);
};

Profiler.prototype.collect = function () {
  var pending = this.pending;
  this.pending = [];
  for (var i = 0; i < pending.length; i++) {
    var tok = pending[i];
    var ms = this.native.eventElapsed(tok.start, tok.stop); // waits for the stop event
    var name = tok.meta.name || "?";
    var s = this.stats.get(name) || { name: name, count: 0, ms: 0, flops: 0 };
    s.count++;
    s.ms += ms;
    s.flops += tok.meta.flops || 0;
    this.stats.set(name, s);
    this.spare.push(tok.start, tok.stop);
  }
};

Profiler.prototype.reset = function () {
  this.stats.clear();
};

// -> Promise<[{ name, count, ms, flops }]>, most time first.
Profiler.prototype.report = function () {
  try {
    this.collect();
  } catch (e) {
    return Promise.reject(e);
  }
  var rows = [];
  this.stats.forEach(function (s) {
    rows.push({ name: s.name, count: s.count, ms: s.ms, flops: s.flops });
  });
  rows.sort(function (a, b) {
    return b.ms - a.ms;
  });
  return Promise.resolve(rows);
};

Profiler.prototype.destroy = function () {
  var self = this;
  this.pending.forEach(function (tok) {
    self.spare.push(tok.start, tok.stop);
  });
  this.pending = [];
  this.spare.forEach(function (ev) {
    self.native.eventDestroy(ev);
  });
  this.spare = [];
};

function lostError(cause) {
  var e = new Error("HIP device lost: " + (cause && cause.message ? cause.message : String(cause)));
  e.code = "SA_ERR_HIP";
  e.cause = cause;
  return e;
}

function GPU(native) {
  this.native = native;
  this.pool = new BufferPool(native);
  this.lost = null;
  this.profiler = null;
}

// GPU.create({ native, profile }) -> Promise<GPU>. Throws a named error (NoDevice) when no HIP
// device is visible, as app/gpu/device.js:92-113 does for a missing adapter or device. With
// profile: true every operator call is timed (gpu.profiler).
GPU.create = function (opts) {
  var native = (opts && opts.native) || loadNative();
  return new Promise(function (resolve, reject) {
    if (native.deviceCount() < 1) {
      var e = new Error("no HIP device is visible");
      e.name = "NoDevice";
      reject(e);
      return;
    }
    var gpu = new GPU(native);
    if (opts && opts.profile) gpu.profiler = new Profiler(native);
    resolve(gpu);
  });
};

// Throws the latched error once the device is lost.
GPU.prototype.check = function () {
  if (this.lost) throw lostError(this.lost);
};

// Runs fn(), a call into the device runtime: refused once the device is lost, latches the device
// as lost when it fails with SA_ERR_HIP.
GPU.prototype.guard = function (fn) {
  this.check();
  try {
    return fn();
  } catch (e) {
    if (e && e.code === "SA_ERR_HIP") this.lost = e;
    throw e;
  }
};

// One operator call: guard(fn), timed under meta = { name, flops } while profiling.
GPU.prototype.op = function (meta, fn) {
  var prof = this.profiler;
  if (!prof) return this.guard(fn);
  return this.guard(function () {
    var tok = prof.begin(meta);
    var r;
    try {
      r = fn();
    } catch (e) {
      prof.cancel(tok);
      throw e;
    }
    prof.end(tok);
    return r;
  });
};

GPU.prototype.empty = function (shape, dtype) {
  this.check();
  var dt = dtype || "f32";
  var bytes = product(shape) * ELEMENT_BYTES[dt];
  var got = this.pool.get(bytes);
  return new Tensor(this, got.buf, shape, got.size, dt);
};

GPU.prototype.fromArray = function (arr, shape) {
  var dt = dtypeOf(arr);
  var sh = shape || [arr.length];
  if (product(sh) !== arr.length) throw new RangeError("shape does not match the array length");
  var t = this.empty(sh, dt);
  var native = this.native;
  try {
    this.guard(function () {
      native.upload(t.buf, arr, 0);
    });
  } catch (e) {
    t.release();
    throw e;
  }
  return t;
};

GPU.prototype.write = function (t, arr, byteOffset) {
  var native = this.native;
  this.guard(function () {
    native.upload(t.buf, arr, byteOffset || 0);
  });
};

// Persistent (non-pooled) buffer holding `arr`.
GPU.prototype.upload = function (arr) {
  var native = this.native;
  return this.guard(function () {
    var buf = native.malloc(Math.max(16, arr.byteLength));
    try {
      native.upload(buf, arr, 0);
    } catch (e) {
      native.free(buf);
      throw e;
    }
    return buf;
  });
};

// -> Promise<Float32Array> of the first `count` elements (all by default).
GPU.prototype.read = function (t, count) {
  var n = count === undefined ? t.size : count;
  var out = t.dtype === "i32" ? new Int32Array(n) : t.dtype === "u8" ? new Uint8Array(n) : new Float32Array(n);
  var native = this.native;
  try {
    this.guard(function () {
      native.download(t.buf, out, 0);
    });
  } catch (e) {
    return Promise.reject(e);
  }
  return Promise.resolve(out);
};

GPU.prototype.flush = function () {};

// Waits for the stream; an asynchronous device error surfaces here (app/gpu/device.js:262-268).
GPU.prototype.sync = function () {
  var native = this.native;
  try {
    this.guard(function () {
      native.sync();
    });
  } catch (e) {
    return Promise.reject(e);
  }
  return Promise.resolve();
};

module.exports = { GPU: GPU, Tensor: Tensor, BufferPool: BufferPool, Profiler: Profiler, loadNative: loadNative,
                   ADDON_PATH: ADDON_PATH };
