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

function GPU(native) {
  this.native = native;
  this.pool = new BufferPool(native);
  this.lost = false;
}

// GPU.create({ native }) -> Promise<GPU>. Throws a named error (NoDevice) when no HIP device is
// visible, as app/gpu/device.js:92-113 does for a missing adapter or device.
GPU.create = function (opts) {
  var native = (opts && opts.native) || loadNative();
  return new Promise(function (resolve, reject) {
    if (native.deviceCount() < 1) {
      var e = new Error("no HIP device is visible");
      e.name = "NoDevice";
      reject(e);
      return;
    }
    resolve(new GPU(native));
  });
};

GPU.prototype.empty = function (shape, dtype) {
  var dt = dtype || "f32";
  var bytes = product(shape) * ELEMENT_BYTES[dt];
  var got = this.pool.get(bytes);
  return new Tensor(this, got.buf, shape, got.size, dt);
};

GPU.prototype.fromArray = function (arr, shape) {
  var dt = dtypeOf(arr);
  var t = this.empty(shape || [arr.length], dt);
  if (product(t.shape) !== arr.length) throw new RangeError("shape does not match the array length");
  this.native.upload(t.buf, arr, 0);
  return t;
};

GPU.prototype.write = function (t, arr, byteOffset) {
  this.native.upload(t.buf, arr, byteOffset || 0);
};

// Persistent (non-pooled) buffer holding `arr`.
GPU.prototype.upload = function (arr) {
  var buf = this.native.malloc(Math.max(16, arr.byteLength));
  this.native.upload(buf, arr, 0);
  return buf;
};

// -> Promise<Float32Array> of the first `count` elements (all by default).
GPU.prototype.read = function (t, count) {
  var n = count === undefined ? t.size : count;
  var out = t.dtype === "i32" ? new Int32Array(n) : t.dtype === "u8" ? new Uint8Array(n) : new Float32Array(n);
  try {
    this.native.download(t.buf, out, 0);
  } catch (e) {
    return Promise.reject(e);
  }
  return Promise.resolve(out);
};

GPU.prototype.flush = function () {};

GPU.prototype.sync = function () {
  try {
    this.native.sync();
  } catch (e) {
    return Promise.reject(e);
  }
  return Promise.resolve();
};

module.exports = { GPU: GPU, Tensor: Tensor, BufferPool: BufferPool, loadNative: loadNative, ADDON_PATH: ADDON_PATH };
