// Safetensors weights for the Supra2-Img Web model loaders, on MI355X: the surface of
// app/weights.js (SafeTensors.open / has / info / f32 / rows, toF32, bf16ToF32, uploadVector,
// uploadLinear, linearFromArray, uploadConv3) over the N-API addon and include/supra_weights.h.
//
// The reference decodes every tensor on the CPU and uploads the Float32Array. Here the file's whole
// data section is copied to device memory once (SafeTensors.prototype.resident: a bulk DMA through
// pinned staging), and every decode, the embedding-row gather and the conv re-layout run on the
// device from that copy. f32() and rows() still return Float32Arrays for callers that want host
// data (dit.js reads pos_embed and the adaLN weights that way); tensor(), rowsTensor() and
// decodeInto() keep results on the device.
//
// Sources: a file path (memory-mapped) or the file's bytes as a Uint8Array/Buffer/ArrayBuffer
// (copied). Errors throw with err.code set to the C ABI status: "SA_ERR_NOT_FOUND" for a missing
// tensor ("missing tensor <name>", as info() throws in the reference), "SA_ERR_FORMAT" for a file
// that is not well-formed safetensors, "SA_ERR_IO", "SA_ERR_UNSUPPORTED" ("unsupported dtype X").
"use strict";

var device = require("./device");

var STAGING_BYTES = 64 << 20; // pinned staging for the bulk upload (two 32 MiB halves)

function codedError(code, msg) {
  var e = new Error(msg);
  e.code = code;
  return e;
}

// dtype name -> addon code for the dtypes toF32 decodes (app/weights.js:4)
function dtypeCodes(native) {
  var out = {};
  ["F32", "F16", "BF16", "F64", "I64", "I32", "I16", "I8", "U8", "BOOL"].forEach(function (n) {
    out[n] = native["SA_DT_" + n];
  });
  return out;
}

function SafeTensors(native, handle) {
  this.native = native;
  this.handle = handle;
  this.metadata = native.stMetadata(handle);
  this.codes = dtypeCodes(native);
  this.gpu = null; // the GPU the data section is resident on
  this.dev = null; // { buf, bytes }
}

// SafeTensors.open(src[, { native }]) -> Promise<SafeTensors> (app/weights.js:40-47)
SafeTensors.open = function (src, opts) {
  var native = (opts && opts.native) || device.loadNative();
  try {
    var h;
    if (typeof src === "string") h = native.stOpen(src);
    else if (src instanceof ArrayBuffer) h = native.stOpenBytes(new Uint8Array(src));
    else if (ArrayBuffer.isView(src)) h = native.stOpenBytes(new Uint8Array(src.buffer, src.byteOffset, src.byteLength));
    else throw codedError("SA_ERR_INVALID", "SafeTensors.open takes a path or the file's bytes");
    return Promise.resolve(new SafeTensors(native, h));
  } catch (e) {
    return Promise.reject(e);
  }
};

SafeTensors.prototype.has = function (name) {
  return this.native.stHas(this.handle, name);
};

// The header entry { dtype, shape, data_offsets } (app/weights.js:60-64).
SafeTensors.prototype.info = function (name) {
  var t = this.native.stInfo(this.handle, name);
  return { dtype: t.dtype, shape: t.shape, data_offsets: t.data_offsets };
};

SafeTensors.prototype.names = function () {
  return this.native.stNames(this.handle);
};

Object.defineProperty(SafeTensors.prototype, "header", {
  get: function () {
    var out = {};
    var self = this;
    this.names().forEach(function (n) {
      out[n] = self.info(n);
    });
    return out;
  },
});

// The data section in device memory on `gpu` (copied on first use; one GPU per file).
SafeTensors.prototype.resident = function (gpu) {
  if (this.dev) {
    if (gpu && gpu !== this.gpu) throw codedError("SA_ERR_INVALID", "the weights are resident on another GPU object");
    return this.dev;
  }
  var g = gpu || this.gpu || new device.GPU(this.native);
  var native = this.native;
  var bytes = native.stDataBytes(this.handle);
  var buf = native.malloc(Math.max(16, bytes));
  var staging = null;
  try {
    if (bytes > 0) {
      var sb = Math.max(2 << 20, Math.min(STAGING_BYTES, 2 * bytes));
      staging = native.mallocHost(sb);
      native.stUpload(this.handle, 0, bytes, buf, 0, staging, sb);
    }
  } catch (e) {
    native.free(buf);
    throw e;
  } finally {
    if (staging) native.freeHost(staging);
  }
  this.gpu = g;
  this.dev = { buf: buf, bytes: bytes };
  return this.dev;
};

// The GPU object the data section lives on (made resident on `gpu`, or on a GPU over the same addon).
SafeTensors.prototype._device = function (gpu) {
  this.resident(gpu);
  return this.gpu;
};

SafeTensors.prototype._entry = function (name) {
  var t = this.native.stInfo(this.handle, name);
  if (this.codes[t.dtype] === undefined) throw codedError("SA_ERR_UNSUPPORTED", "unsupported dtype " + t.dtype);
  return t;
};

// Decodes tensor `name` into the device buffer `dst` at byte offset `dstByteOffset` (float32).
SafeTensors.prototype.decodeInto = function (gpu, name, dst, dstByteOffset) {
  var t = this._entry(name);
  var dev = this.resident(gpu);
  var native = this.native;
  var code = this.codes[t.dtype];
  this.gpu.op({ name: "toF32", flops: 0 }, function () {
    native.toF32(dev.buf, t.data_offsets[0], code, t.numel, dst, dstByteOffset || 0);
  });
  return t.numel;
};

// tensor(gpu, name) -> pooled float32 Tensor of the tensor's shape, decoded on the device.
SafeTensors.prototype.tensor = function (gpu, name) {
  var t = this._entry(name);
  var g = this._device(gpu);
  var out = g.empty(t.shape.length ? t.shape : [1]);
  this.decodeInto(g, name, out.buf, 0);
  return out;
};

// f32(name) -> Promise<Float32Array> (app/weights.js:66-70)
SafeTensors.prototype.f32 = function (name) {
  try {
    var g = this._device(null);
    var t = this.tensor(g, name);
    return g.read(t, t.size).then(function (a) {
      t.release();
      return a;
    });
  } catch (e) {
    return Promise.reject(e);
  }
};

// rowsTensor(gpu, name, ids) -> pooled [ids.length, dim] float32 Tensor (ids outside the table
// give zero rows).
SafeTensors.prototype.rowsTensor = function (gpu, name, ids) {
  var t = this._entry(name);
  if (t.shape.length !== 2) throw codedError("SA_ERR_INVALID", name + " is not a 2-D table");
  var dim = t.shape[1];
  var g = this._device(gpu);
  var dev = this.dev;
  var out = g.empty([ids.length, dim]);
  if (ids.length) {
    var idt = g.fromArray(Int32Array.from(ids));
    var native = this.native;
    var code = this.codes[t.dtype];
    try {
      g.op({ name: "rowsF32", flops: 0 }, function () {
        native.rowsF32(dev.buf, t.data_offsets[0], code, t.shape[0], dim, idt.buf, ids.length, out.buf);
      });
    } finally {
      idt.release();
    }
  }
  return out;
};

// rows(name, ids) -> Promise<Float32Array> of ids.length * dim (app/weights.js:73-83)
SafeTensors.prototype.rows = function (name, ids) {
  try {
    var g = this._device(null);
    var t = this.rowsTensor(g, name, ids);
    return g.read(t, t.size).then(function (a) {
      t.release();
      return a;
    });
  } catch (e) {
    return Promise.reject(e);
  }
};

SafeTensors.prototype.close = function () {
  if (this.dev) {
    this.native.free(this.dev.buf);
    this.dev = null;
  }
  if (this.handle) {
    this.native.stClose(this.handle);
    this.handle = null;
  }
};

// A persistent float32 device buffer holding tensor `name` (like gpu.upload(await src.f32(name))).
function persistent(gpu, src, name) {
  var t = src._entry(name);
  var buf = gpu.native.malloc(Math.max(16, t.numel * 4));
  src.decodeInto(gpu, name, buf, 0);
  return buf;
}

// uploadVector(gpu, src, name) -> Promise<device buffer> (app/weights.js:85-87)
function uploadVector(gpu, src, name) {
  try {
    return Promise.resolve(persistent(gpu, src, name));
  } catch (e) {
    return Promise.reject(e);
  }
}

// uploadLinear(gpu, src, base) -> Promise<{ kind, N, K, buf, bias }> (app/weights.js:89-96)
function uploadLinear(gpu, src, base) {
  try {
    var w = src.info(base + "weight");
    var N = w.shape[0];
    var K = w.shape.slice(1).reduce(function (a, b) {
      return a * b;
    }, 1);
    var bias = src.has(base + "bias") ? persistent(gpu, src, base + "bias") : null;
    return Promise.resolve({ kind: "f32", N: N, K: K, buf: persistent(gpu, src, base + "weight"), bias: bias });
  } catch (e) {
    return Promise.reject(e);
  }
}

// linearFromArray(gpu, data, N, K, bias) (app/weights.js:98-101)
function linearFromArray(gpu, data, N, K, bias) {
  return { kind: "f32", N: N, K: K, buf: gpu.upload(data), bias: bias ? gpu.upload(bias) : null };
}

// uploadConv3(gpu, src, base, cinPad) -> Promise<{ kind, N: cout, K: 9 * cinPad, buf, bias }>
// (app/weights.js:105-118): [cout, cin, 3, 3] -> [cout, 3, 3, cinPad] on the device.
function uploadConv3(gpu, src, base, cinPad) {
  try {
    var t = src._entry(base + "weight");
    var s = t.shape;
    if (s.length !== 4 || s[2] !== 3 || s[3] !== 3) throw codedError("SA_ERR_INVALID", base + ": expected a 3x3 conv");
    var cout = s[0];
    var cin = s[1];
    var cp = cinPad || cin;
    var dev = src.resident(gpu);
    var buf = gpu.native.malloc(Math.max(16, cout * 9 * cp * 4));
    try {
      gpu.op({ name: "conv3Pack", flops: 0 }, function () {
        gpu.native.conv3Pack(dev.buf, t.data_offsets[0], src.codes[t.dtype], cout, cin, cp, buf);
      });
    } catch (e) {
      gpu.native.free(buf);
      throw e;
    }
    var bias = src.has(base + "bias") ? persistent(gpu, src, base + "bias") : null;
    return Promise.resolve({ kind: "f32", N: cout, K: 9 * cp, buf: buf, bias: bias });
  } catch (e) {
    return Promise.reject(e);
  }
}

var defaultGpu = null;

// toF32(u8, dtype) -> Float32Array (app/weights.js:28-37), decoded on the device.
function toF32(u8, dtype, opts) {
  var native = (opts && opts.native) || device.loadNative();
  var codes = dtypeCodes(native);
  if (codes[dtype] === undefined) throw codedError("SA_ERR_UNSUPPORTED", "unsupported dtype " + dtype);
  if (!defaultGpu || defaultGpu.native !== native) defaultGpu = new device.GPU(native);
  var g = defaultGpu;
  var bytes = new Uint8Array(u8.buffer, u8.byteOffset, u8.byteLength);
  var esize = { F64: 8, F32: 4, BF16: 2, F16: 2, I64: 8, I32: 4, I16: 2, I8: 1, U8: 1, BOOL: 1 }[dtype];
  var n = Math.floor(bytes.byteLength / esize);
  var src = g.fromArray(bytes);
  var out = g.empty([Math.max(1, n)]);
  var res = new Float32Array(n);
  try {
    native.toF32(src.buf, 0, codes[dtype], n, out.buf, 0);
    if (n) native.download(out.buf, res, 0);
  } finally {
    src.release();
    out.release();
  }
  return res;
}

function bf16ToF32(u8) {
  return toF32(u8, "BF16");
}

module.exports = {
  SafeTensors: SafeTensors,
  uploadVector: uploadVector,
  uploadLinear: uploadLinear,
  linearFromArray: linearFromArray,
  uploadConv3: uploadConv3,
  toF32: toF32,
  bf16ToF32: bf16ToF32,
};
