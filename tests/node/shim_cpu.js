// CPU checks of the JS binding (no GPU): the addon loads under Node, exports its functions and
// constants, computes T5 buckets, rejects invalid calls with C ABI status codes; the shim maps the
// reference call forms (app/models/dit.js:172, dit.js:184, t5.js:80, vae.js:86) onto sa_attn_args
// as expected, and the buffer pool reuses released buffers.
// Usage: node tests/node/shim_cpu.js <expected-buckets.json>
"use strict";

var assert = require("assert");
var fs = require("fs");
var path = require("path");

var root = path.join(__dirname, "..", "..", "supra2-img-web_amd", "js");
var sa = require(path.join(root, "index.js"));
var device = require(path.join(root, "device.js"));
var native = device.loadNative();

var checks = 0;
var pending = [];
function check(name, fn) {
  fn();
  checks++;
  process.stdout.write("ok " + name + "\n");
}

check("addon exports", function () {
  ["attention", "kernelName", "workspaceBytes", "version", "deviceCount", "malloc", "free", "upload", "download", "memset", "copy", "sync", "linear", "linearKernelName", "vaeAttention", "vaeWorkspaceBytes",
    "bucketLut", "positionBias", "eventCreate", "eventRecord", "eventElapsed", "eventDestroy"].forEach(function (f) {
    assert.strictEqual(typeof native[f], "function", f);
  });
  assert.strictEqual(native.version(), 5);
  assert.strictEqual(native.SA_BIAS_RELPOS, 2);
  assert.strictEqual(native.SA_MASK_KEY_MASK, 2);
});

check("handles: only this addon's, of the right kind, and live", function () {
  var invalid = function (re) {
    return function (e) { return e.code === "SA_ERR_INVALID" && re.test(e.message); };
  };
  // not a handle at all: plain objects, numbers, typed arrays
  assert.throws(function () { native.upload({}, new Float32Array(4), 0); }, invalid(/buffer must be a device buffer handle/));
  assert.throws(function () { native.free(12345); }, invalid(/buffer must be a device buffer handle/));
  assert.throws(function () { native.copy(new Float32Array(4), 0, null, 0, 16); }, invalid(/dst must be a device buffer/));
  assert.throws(function () {
    native.attention({ B: 1, H: 1, D: 64, Lq: 4, Lk: 4, q: { buf: 1 }, ldq: 64, ldk: 64, ldv: 64 });
  }, invalid(/q must be a device buffer handle/));
  assert.throws(function () { native.eventRecord({}); }, invalid(/event must be an event handle/));
  // a handle of another kind: an opened file where a device buffer or an event belongs
  var bytes = fs.readFileSync(JSON.parse(fs.readFileSync(process.argv[3], "utf8")).file);
  var f = native.stOpenBytes(new Uint8Array(bytes.buffer, bytes.byteOffset, bytes.length));
  assert.throws(function () { native.upload(f, new Float32Array(4), 0); }, invalid(/device buffer handle/));
  assert.throws(function () { native.linear({ M: 1, N: 1, K: 8, x: f }); }, invalid(/x must be a device buffer handle/));
  assert.throws(function () { native.eventDestroy(f); }, invalid(/event handle/));
  assert.throws(function () { native.freeHost(f); }, invalid(/pinned host buffer handle/));
  assert.ok(native.stNames(f).length > 0);
  // released: a closed file throws on use, closing again is allowed
  native.stClose(f);
  assert.throws(function () { native.stNames(f); }, invalid(/has been released/));
  native.stClose(f);
  assert.throws(function () { native.stClose({}); }, invalid(/safetensors handle/));
});

check("bucket LUT matches the oracle's", function () {
  var expected = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  var lut = native.bucketLut(expected.Lq, expected.Lk, 32, 128, true);
  assert.strictEqual(lut.length, expected.lut.length);
  for (var i = 0; i < lut.length; i++) assert.strictEqual(lut[i], expected.lut[i], "index " + i);
  expected.singles.forEach(function (p) {
    assert.strictEqual(sa.relativeBucket(p[0], 32, 128, native), p[1], "rel " + p[0]);
  });
});

check("invalid calls throw with a status code before touching the device", function () {
  assert.throws(function () {
    native.attention({ B: 1, H: 1, D: 64, Lq: 4, Lk: 4, ldq: 64, ldk: 64, ldv: 64, scale: 1 });
  }, function (e) {
    return e.code === "SA_ERR_INVALID" && /non-NULL/.test(e.message);
  });
  assert.throws(function () {
    native.attention({ H: 2, D: 64, Lq: "x" });
  }, function (e) {
    return e.code === "SA_ERR_INVALID";
  });
  assert.throws(function () {
    native.bucketLut(0, 4, 32, 128, true);
  }, function (e) {
    return e.code === "SA_ERR_INVALID";
  });
  // the host copy of the key lengths must be an Int32Array of at least B entries (it is read on the host)
  [[77, 1], new Float32Array(2), new Int32Array(1)].forEach(function (klh) {
    assert.throws(function () {
      native.attention({ B: 2, H: 9, D: 64, Lq: 256, Lk: 128, ldq: 576, ldk: 1152, ldv: 1152, keyLenHost: klh });
    }, function (e) {
      return e.code === "SA_ERR_INVALID" && /keyLenHost must be an Int32Array of at least B lengths/.test(e.message);
    });
  });
});

// a fake addon: records calls, hands out numbered buffers
function fakeNative() {
  var n = 0;
  return {
    calls: [],
    mallocs: 0,
    deviceCount: function () { return 1; },
    malloc: function (bytes) { this.mallocs++; return { id: ++n, bytes: bytes }; },
    free: function () { this.frees++; },
    upload: function () {},
    copies: [],
    copy: function (dst, doff, src, soff, bytes) { this.copies.push([dst, doff, src, soff, bytes]); },
    download: function () {},
    sync: function () {},
    attention: function (a) { this.calls.push(a); },
    lin: [],
    linear: function (a) { this.lin.push(a); },
    vae: [],
    vaeAttention: function (a) { this.vae.push(a); },
    vaeWorkspaceBytes: function () { return 27328512; },
    kernelName: function () { return "fake"; },
    wsBytes: 0,
    frees: 0,
    workspaceBytes: function () { return this.wsBytes; },
    bucketLut: native.bucketLut,
  };
}

function makeGpu() {
  var f = fakeNative();
  return { f: f, gpu: new device.GPU(f) };
}

check("DiT self-attention form (dit.js:172)", function () {
  var g = makeGpu();
  var D = 576, TOK = 256;
  var qkv = g.gpu.empty([2 * TOK, 3 * D]);
  var a = g.gpu.empty([2 * TOK, D]);
  for (var b = 0; b < 2; b++) {
    var r = b * TOK * 3 * D;
    var ret = sa.attention(g.gpu, { q: qkv, k: qkv, v: qkv, Lq: TOK, Lk: TOK, H: 9, D: 64, ldq: 3 * D, ldk: 3 * D,
      ldv: 3 * D, qOff: r, kOff: r + D, vOff: r + 2 * D, oOff: b * TOK * D, out: a });
    assert.strictEqual(ret, a);
  }
  assert.strictEqual(g.f.calls.length, 2);
  var c = g.f.calls[1];
  assert.strictEqual(c.B, 1);
  assert.strictEqual(c.qOff, TOK * 3 * D);
  assert.strictEqual(c.kOff, TOK * 3 * D + D);
  assert.strictEqual(c.vOff, TOK * 3 * D + 2 * D);
  assert.strictEqual(c.oOff, TOK * D);
  assert.strictEqual(c.ldo, D);
  assert.strictEqual(c.scale, 1 / 8);
  assert.strictEqual(c.q, qkv.buf);
  assert.strictEqual(c.out, a.buf);
  assert.strictEqual(c.biasMode, 0);
  assert.strictEqual(c.maskMode, 0);
});

check("DiT cross-attention form (dit.js:184) and its batched padded form", function () {
  var g = makeGpu();
  var q = g.gpu.empty([512, 576]);
  var kv = g.gpu.empty([77, 1152]);
  var c = g.gpu.empty([512, 576]);
  sa.attention(g.gpu, { q: q, k: kv, v: kv, Lq: 256, Lk: 77, H: 9, D: 64, ldq: 576, ldk: 1152, ldv: 1152,
    qOff: 256 * 576, kOff: 0, vOff: 576, oOff: 256 * 576, out: c });
  var a = g.f.calls[0];
  assert.strictEqual(a.Lk, 77);
  assert.strictEqual(a.vOff, 576);
  assert.strictEqual(a.ldk, 1152);
  var kvp = g.gpu.empty([2 * 128, 1152]);
  var kl = g.gpu.fromArray(new Int32Array([77, 1]), [2]);
  sa.attention(g.gpu, { B: 2, q: q, k: kvp, v: kvp, Lq: 256, Lk: 128, H: 9, D: 64, ldq: 576, ldk: 1152, ldv: 1152,
    vOff: 576, sq: 256 * 576, sk: 128 * 1152, sv: 128 * 1152, so: 256 * 576, keyLen: kl, out: c });
  a = g.f.calls[1];
  assert.strictEqual(a.B, 2);
  assert.strictEqual(a.maskMode, 1);
  assert.strictEqual(a.keyLen, kl.buf);
  assert.strictEqual(a.sk, 128 * 1152);
  assert.strictEqual(kl.dtype, "i32");
});

check("T5 form (t5.js:80): scale 1, dense bias; relpos + key-mask extension", function () {
  var g = makeGpu();
  var q = g.gpu.empty([128, 768]);
  var bias = g.gpu.empty([12, 128, 128]);
  var out = sa.attention(g.gpu, { q: q, k: q, v: q, Lq: 128, Lk: 128, H: 12, D: 64, ldq: 768, ldk: 768, ldv: 768,
    scale: 1, bias: bias });
  assert.deepStrictEqual(out.shape, [128, 768]);
  var a = g.f.calls[0];
  assert.strictEqual(a.scale, 1);
  assert.strictEqual(a.biasMode, 1);
  assert.strictEqual(a.bias, bias.buf);
  assert.strictEqual(a.sbias, 0);
  var rp = sa.relposBias(g.gpu, new Float32Array(32 * 12), 32, 12, 128, 128);
  assert.deepStrictEqual(rp.lut.shape, [255]);
  var km = g.gpu.fromArray(new Uint8Array(128).fill(1), [1, 128]);
  sa.attention(g.gpu, { q: q, k: q, v: q, Lq: 128, Lk: 128, H: 12, D: 64, ldq: 768, ldk: 768, ldv: 768, scale: 1,
    relpos: rp, keyMask: km });
  a = g.f.calls[1];
  assert.strictEqual(a.biasMode, 2);
  assert.strictEqual(a.numBuckets, 32);
  assert.strictEqual(a.bucketLut, rp.lut.buf);
  assert.strictEqual(a.maskMode, 2);
  assert.strictEqual(a.smask, 128);
});

check("VAE form (vae.js:86): one head, D = 512, default scale", function () {
  var g = makeGpu();
  var q = g.gpu.empty([1024, 512]);
  sa.attention(g.gpu, { q: q, k: q, v: q, Lq: 1024, Lk: 1024, H: 1, D: 512, ldq: 512, ldk: 512, ldv: 512 });
  var a = g.f.calls[0];
  assert.strictEqual(a.scale, 1 / Math.sqrt(512));
  assert.strictEqual(a.ldo, 512);
  assert.strictEqual(a.so, 512 * 1024);
  assert.strictEqual(a.workspace, undefined);
  // a call that needs device scratch gets a pooled buffer, returned to the pool after the launch
  g.f.wsBytes = 16805888;
  sa.attention(g.gpu, { q: q, k: q, v: q, Lq: 1024, Lk: 1024, H: 1, D: 512, ldq: 512, ldk: 512, ldv: 512 });
  var w = g.f.calls[1];
  assert.strictEqual(w.workspaceBytes, 16805888);
  assert.ok(w.workspace && w.workspace.bytes >= 16805888);
  var before = g.f.mallocs;
  var again = g.gpu.empty([16805888 / 4]);
  assert.strictEqual(again.buf, w.workspace);
  assert.strictEqual(g.f.mallocs, before);
  // the workspace goes back to the pool when the launch throws, too
  g.f.attention = function () { throw new Error("launch failed"); };
  again.release();
  assert.throws(function () {
    sa.attention(g.gpu, { q: q, k: q, v: q, Lq: 1024, Lk: 1024, H: 1, D: 512, ldq: 512, ldk: 512, ldv: 512 });
  }, /launch failed/);
  assert.strictEqual(g.gpu.empty([16805888 / 4]).buf, w.workspace);
});

check("batched DiT call sites: one launch per block (dit.js:169-173, 180-185)", function () {
  var g = makeGpu();
  var D = 576, TOK = 256, B = 4;
  var qkv = g.gpu.empty([B * TOK, 3 * D]);
  var a = sa.dit.selfAttention(g.gpu, qkv, B);
  assert.strictEqual(g.f.calls.length, 1);
  var s = g.f.calls[0];
  assert.strictEqual(s.B, B);
  assert.strictEqual(s.q, qkv.buf);
  assert.strictEqual(s.kOff, D);
  assert.strictEqual(s.vOff, 2 * D);
  assert.strictEqual(s.sq, TOK * 3 * D);
  assert.strictEqual(s.so, TOK * D);
  assert.deepStrictEqual(a.shape, [B * TOK, D]);
  var lens = [77, 1, 50, 0];
  var kvs = lens.map(function (L) { return g.gpu.empty([Math.max(L, 1), 2 * D]); });
  var ctx = sa.dit.packContexts(g.gpu, kvs, lens);
  assert.strictEqual(ctx.Lmax, 77);
  assert.strictEqual(g.f.copies.length, 3);  // the empty context copies nothing
  assert.deepStrictEqual(g.f.copies[1], [ctx.kv.buf, 1 * 77 * 2 * D * 4, kvs[1].buf, 0, 1 * 2 * D * 4]);
  assert.deepStrictEqual(g.f.copies[2], [ctx.kv.buf, 2 * 77 * 2 * D * 4, kvs[2].buf, 0, 50 * 2 * D * 4]);
  var q = g.gpu.empty([B * TOK, D]);
  sa.dit.crossAttention(g.gpu, q, ctx);
  assert.strictEqual(g.f.calls.length, 2);
  var c = g.f.calls[1];
  assert.strictEqual(c.B, B);
  assert.strictEqual(c.Lk, 77);
  assert.strictEqual(c.keyLen, ctx.keyLen.buf);
  assert.strictEqual(c.vOff, D);
  assert.strictEqual(c.sk, 77 * 2 * D);
  assert.strictEqual(c.ldk, 2 * D);
  ctx.release();
  assert.strictEqual(ctx.kv.buf, null);
  assert.throws(function () { sa.dit.packContexts(g.gpu, kvs, [1, 2]); }, RangeError);
});

check("linear forms of the DiT block (dit.js:167, 175, 191; ops.js:35-43)", function () {
  var g = makeGpu();
  var R = 512, D = 576;
  var h = g.gpu.empty([R, D]);
  var Wqkv = { kind: "f32", N: 3 * D, K: D, buf: g.gpu.upload(new Float32Array(16)), bias: g.gpu.upload(new Float32Array(4)) };
  var qkv = sa.linear(g.gpu, h, Wqkv);
  assert.deepStrictEqual(qkv.shape, [R, 3 * D]);
  var a = g.f.lin[0];
  assert.strictEqual(a.M, R);
  assert.strictEqual(a.N, 3 * D);
  assert.strictEqual(a.K, D);
  assert.strictEqual(a.w, Wqkv.buf);
  assert.strictEqual(a.bias, Wqkv.bias);
  assert.strictEqual(a.act, 0);
  assert.strictEqual(a.epilogue, 0);
  assert.strictEqual(a.y, qkv.buf);
  // proj: out += gate[gOff + n] * (a W^T + b)
  var x = g.gpu.empty([R, D]);
  var mod = g.gpu.empty([1, 14 * 6 * D]);
  var Wp = { kind: "f32", N: D, K: D, buf: g.gpu.upload(new Float32Array(16)), bias: null };
  var ret = sa.linear(g.gpu, h, Wp, { out: x, resid: true, gate: mod, gOff: 2 * D });
  assert.strictEqual(ret, x);
  a = g.f.lin[1];
  assert.strictEqual(a.epilogue, 2);
  assert.strictEqual(a.gate, mod.buf);
  assert.strictEqual(a.gateOff, 2 * D);
  assert.strictEqual(a.bias, null);
  // fc1 with GELU (tanh), cproj residual without a gate, rows/aOff
  sa.linear(g.gpu, h, Wp, { act: "gelu_tanh" });
  assert.strictEqual(g.f.lin[2].act, 2);
  sa.linear(g.gpu, h, Wp, { out: x, resid: true });
  assert.strictEqual(g.f.lin[3].epilogue, 1);
  sa.linear(g.gpu, h, Wp, { rows: 100, aOff: 7 * D });
  assert.strictEqual(g.f.lin[4].M, 100);
  assert.strictEqual(g.f.lin[4].xOff, 7 * D);
  assert.throws(function () { sa.linear(g.gpu, h, Wp, { act: "relu6" }); }, /unknown act/);
  assert.throws(function () { sa.linear(g.gpu, h, { kind: "q8", N: D, K: D, buf: Wp.buf }); }, /f32/);
  h.release();
  assert.throws(function () { sa.linear(g.gpu, h, Wp); }, /released/);
});

check("VAE mid-block attention (vae.js:77-94) as one call", function () {
  var g = makeGpu();
  var C = 512;
  var lin = function () { return { kind: "f32", N: C, K: C, buf: g.gpu.upload(new Float32Array(4)), bias: g.gpu.upload(new Float32Array(4)) }; };
  var A = { norm: { g: g.gpu.upload(new Float32Array(4)), b: g.gpu.upload(new Float32Array(4)) }, q: lin(), k: lin(), v: lin(), o: lin() };
  var x = g.gpu.empty([1024, C]);
  var ret = sa.vae.attention(g.gpu, x, 1024, A);
  assert.strictEqual(ret, x);  // consumed and overwritten, as the reference's attention() consumes x
  assert.strictEqual(g.f.copies.length, 6);  // q, k, v weights and biases packed once
  var a = g.f.vae[0];
  assert.strictEqual(a.HW, 1024);
  assert.strictEqual(a.C, C);
  assert.strictEqual(a.groups, 32);
  assert.strictEqual(a.out, x.buf);
  assert.strictEqual(a.x, x.buf);
  assert.strictEqual(a.wo, A.o.buf);
  assert.strictEqual(a.workspaceBytes, 27328512);
  assert.deepStrictEqual(g.f.copies[2], [a.wqkv, C * C * 4, A.k.buf, 0, C * C * 4]);  // q.w, q.b, k.w, ...
  assert.deepStrictEqual(g.f.copies[3], [a.bqkv, C * 4, A.k.bias, 0, C * 4]);
  sa.vae.attention(g.gpu, x, 1024, A);
  assert.strictEqual(g.f.copies.length, 6);  // cached
  A.k.bias = null;
  A._saQkv = null;
  assert.throws(function () { sa.vae.attention(g.gpu, x, 1024, A); }, /biases or none/);
});

check("released tensors are reused and cannot be passed again", function () {
  var g = makeGpu();
  var t = g.gpu.empty([1000]);
  var buf = t.buf;
  t.release();
  assert.strictEqual(t.buf, null);
  var u = g.gpu.empty([999]);
  assert.strictEqual(u.buf, buf);
  assert.strictEqual(g.f.mallocs, 1);
  assert.throws(function () {
    sa.attention(g.gpu, { q: t, k: u, v: u, Lq: 1, Lk: 1, H: 1, D: 64, ldq: 64, ldk: 64, ldv: 64 });
  }, /released/);
  assert.strictEqual(device.BufferPool.round(1), 256);
  assert.strictEqual(device.BufferPool.round(5000), 5120);
});

// a fake addon with HIP events: elapsed time = difference of record counters (ms)
function timedNative() {
  var f = fakeNative();
  var clock = 0, ev = 0;
  f.created = 0;
  f.destroyed = 0;
  f.eventCreate = function () { f.created++; return { ev: ++ev, t: null }; };
  f.eventRecord = function (e) { clock += 1; e.t = clock; };
  f.eventElapsed = function (a, b) { return b.t - a.t; };
  f.eventDestroy = function () { f.destroyed++; };
  f.attention = function (a) { clock += 10; this.calls.push(a); };
  f.linear = function (a) { clock += 100; this.lin.push(a); };
  return f;
}

checkAsync("profiler: per-operator ms and flops (app/gpu/device.js:272-325)", function () {
  var f = timedNative();
  return device.GPU.create({ native: f, profile: true }).then(function (gpu) {
    assert.ok(gpu.profiler instanceof device.Profiler);
    var q = gpu.empty([256 * 2, 1728]);
    sa.attention(gpu, { q: q, k: q, v: q, B: 2, Lq: 256, Lk: 256, H: 9, D: 64, ldq: 1728, ldk: 1728, ldv: 1728,
                        kOff: 576, vOff: 1152, sq: 256 * 1728, sk: 256 * 1728, sv: 256 * 1728 });
    sa.attention(gpu, { q: q, k: q, v: q, B: 2, Lq: 256, Lk: 256, H: 9, D: 64, ldq: 1728, ldk: 1728, ldv: 1728,
                        kOff: 576, vOff: 1152, sq: 256 * 1728, sk: 256 * 1728, sv: 256 * 1728 });
    var W = { kind: "f32", N: 1728, K: 576, buf: gpu.empty([1728, 576]), bias: null };
    sa.linear(gpu, gpu.empty([512, 576]), W);
    // a call rejected before its launch is not counted
    f.attention = function () { var e = new Error("bad"); e.code = "SA_ERR_INVALID"; throw e; };
    assert.throws(function () {
      sa.attention(gpu, { q: q, k: q, v: q, Lq: 1, Lk: 1, H: 1, D: 64, ldq: 64, ldk: 64, ldv: 64 });
    }, /bad/);
    return gpu.profiler.report().then(function (rows) {
      assert.strictEqual(rows.length, 2);
      assert.strictEqual(rows[0].name, "linear");  // most time first
      assert.strictEqual(rows[0].count, 1);
      assert.strictEqual(rows[0].ms, 101);
      assert.strictEqual(rows[0].flops, 2 * 512 * 1728 * 576);
      assert.strictEqual(rows[1].name, "attention");
      assert.strictEqual(rows[1].count, 2);
      assert.strictEqual(rows[1].ms, 22);
      assert.strictEqual(rows[1].flops, 2 * 4 * 2 * 256 * 256 * 64 * 9);  // 4 Lq Lk D H per sequence (ops.js:116)
      gpu.profiler.reset();
      return gpu.profiler.report();
    }).then(function (rows) {
      assert.strictEqual(rows.length, 0);
      gpu.profiler.destroy();
      assert.strictEqual(f.destroyed, f.created);  // events are recycled, then all destroyed
      assert.strictEqual(f.created, 7);  // three timed calls + the start of the rejected one
    });
  });
});

checkAsync("profiler: key-length calls count attended keys (app/gpu/ops.js:116 with each sample's own Lk)", function () {
  var f = timedNative();
  return device.GPU.create({ native: f, profile: true }).then(function (gpu) {
    var q = gpu.empty([4 * 256, 576]);
    var kv = gpu.empty([4 * 128, 1152]);
    var kl = gpu.empty([4], "i32");
    var lens = new Int32Array([77, 1, 200, -3]);  // clamped to [0, Lk]: 77 + 1 + 128 + 0 keys
    var base = { q: q, k: kv, v: kv, B: 4, Lq: 256, Lk: 128, H: 9, D: 64, ldq: 576, ldk: 1152, ldv: 1152,
                 kOff: 0, vOff: 576, sq: 256 * 576, sk: 128 * 1152, sv: 128 * 1152, keyLen: kl };
    sa.attention(gpu, Object.assign({ keyLenHost: lens }, base));
    return gpu.profiler.report().then(function (rows) {
      assert.strictEqual(rows[0].flops, 4 * 256 * (77 + 1 + 128 + 0) * 64 * 9);
      gpu.profiler.reset();
      sa.attention(gpu, base);  // no host copy: the padded length
      return gpu.profiler.report();
    }).then(function (rows) {
      assert.strictEqual(rows[0].flops, 4 * 256 * 4 * 128 * 64 * 9);
      gpu.profiler.reset();
      // the batched DiT helper hands its host lengths over: the count is the per-sample calls' sum
      var ctx = { kv: kv, keyLen: kl, lens: new Int32Array([77, 1, 5, 128]), B: 4, Lmax: 128 };
      sa.dit.crossAttention(gpu, q, ctx);
      return gpu.profiler.report();
    }).then(function (rows) {
      var att = rows.filter(function (r) { return r.name === "attention"; })[0];
      assert.strictEqual(att.flops, 4 * 256 * (77 + 1 + 5 + 128) * 64 * 9);
      gpu.profiler.destroy();
    });
  });
});

checkAsync("device-lost latch: a HIP error makes every later call throw (app/gpu/device.js:134, 208)", function () {
  var f = fakeNative();
  var gpu = new device.GPU(f);
  var q = gpu.empty([64, 64]);
  var args = { q: q, k: q, v: q, Lq: 64, Lk: 64, H: 1, D: 64, ldq: 64, ldk: 64, ldv: 64 };
  // an invalid-argument error does not mark the device lost
  f.attention = function () { var e = new Error("bad stride"); e.code = "SA_ERR_INVALID"; throw e; };
  assert.throws(function () { sa.attention(gpu, args); }, /bad stride/);
  assert.strictEqual(gpu.lost, null);
  f.attention = function () { var e = new Error("hipErrorLaunchFailure"); e.code = "SA_ERR_HIP"; throw e; };
  assert.throws(function () { sa.attention(gpu, args); }, /hipErrorLaunchFailure/);
  assert.ok(gpu.lost);
  var launches = 0;
  f.attention = function () { launches++; };
  assert.throws(function () { sa.attention(gpu, args); }, function (e) {
    return e.code === "SA_ERR_HIP" && /device lost: hipErrorLaunchFailure/.test(e.message);
  });
  assert.throws(function () { gpu.empty([4]); }, /device lost/);
  assert.strictEqual(launches, 0);
  // errors reported at sync latch too, and read/sync reject once lost
  var g2 = new device.GPU(fakeNative());
  g2.native.sync = function () { var e = new Error("async fault"); e.code = "SA_ERR_HIP"; throw e; };
  return g2.sync().then(function () { assert.fail("sync resolved"); }, function (e) {
    assert.ok(/async fault/.test(e.message));
    assert.ok(g2.lost);
    return gpu.read(q).then(function () { assert.fail("read resolved"); }, function (e2) {
      assert.ok(/device lost/.test(e2.message));
    });
  });
});

check("fromArray checks the shape before taking a pooled buffer", function () {
  var g = makeGpu();
  assert.throws(function () { g.gpu.fromArray(new Float32Array(10), [3, 3]); }, /shape does not match/);
  assert.strictEqual(g.f.mallocs, 0);
  // an upload that fails returns its buffer to the pool
  g.f.upload = function () { throw new Error("upload failed"); };
  assert.throws(function () { g.gpu.fromArray(new Float32Array(10), [10]); }, /upload failed/);
  g.f.upload = function () {};
  var t = g.gpu.fromArray(new Float32Array(10), [2, 5]);
  assert.strictEqual(g.f.mallocs, 1);
  assert.deepStrictEqual(t.shape, [2, 5]);
});

function checkAsync(name, fn) {
  pending.push(function () {
    return Promise.resolve(fn()).then(function () {
      checks++;
      process.stdout.write("ok " + name + "\n");
    });
  });
}

checkAsync("safetensors header and errors through the addon (app/weights.js:40-64), host only", function () {
  var exp = JSON.parse(fs.readFileSync(process.argv[3], "utf8"));
  var W = sa.weights;
  return W.SafeTensors.open(exp.file).then(function (st) {
    assert.deepStrictEqual(st.names(), Object.keys(exp.header));
    Object.keys(exp.header).forEach(function (n) {
      assert.ok(st.has(n), n);
      assert.deepStrictEqual(st.info(n), exp.header[n]);
    });
    assert.deepStrictEqual(st.metadata, exp.metadata);
    assert.deepStrictEqual(Object.keys(st.header), Object.keys(exp.header));
    assert.strictEqual(st.has("nope"), false);
    assert.throws(function () { st.info("nope"); }, function (e) {
      return e.code === "SA_ERR_NOT_FOUND" && /missing tensor nope/.test(e.message);
    });
    // checks that precede any device work
    assert.throws(function () { st._entry("u16"); }, function (e) {
      return e.code === "SA_ERR_UNSUPPORTED" && /unsupported dtype U16/.test(e.message);
    });
    return W.uploadConv3(null, st, "blocks.0.mlp.0.", 0).then(function () { assert.fail("conv of a linear"); }, function (e) {
      assert.ok(/expected a 3x3 conv/.test(e.message), e.message);
      st.close();
      assert.throws(function () { st.names(); }, /closed|safetensors handle/);
    });
  }).then(function () {
    var bytes = fs.readFileSync(exp.file);
    return W.SafeTensors.open(bytes).then(function (st) {
      assert.deepStrictEqual(st.names(), Object.keys(exp.header));
      st.close();
    });
  }).then(function () {
    return W.SafeTensors.open(new Uint8Array([5, 0, 0])).then(function () { assert.fail("opened"); }, function (e) {
      assert.strictEqual(e.code, "SA_ERR_FORMAT");
    });
  }).then(function () {
    return W.SafeTensors.open(exp.file + ".missing").then(function () { assert.fail("opened"); }, function (e) {
      assert.strictEqual(e.code, "SA_ERR_IO");
    });
  }).then(function () {
    assert.throws(function () { W.toF32(new Uint8Array(4), "U32"); }, /unsupported dtype U32/);
    assert.strictEqual(native.SA_DT_BF16, 3);
    ["stOpen", "stOpenBytes", "stClose", "stNames", "stInfo", "stHas", "stMetadata", "stDataBytes", "stUpload",
      "mallocHost", "freeHost", "toF32", "rowsF32", "conv3Pack"].forEach(function (f) {
      assert.strictEqual(typeof native[f], "function", f);
    });
  });
});

pending.reduce(function (p, f) { return p.then(f); }, Promise.resolve()).then(function () {
  process.stdout.write("all " + checks + " checks passed\n");
}, function (e) {
  process.stderr.write("check failed: " + (e && e.stack ? e.stack : e) + "\n");
  process.exit(1);
});
