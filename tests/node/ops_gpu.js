// GPU run of the JS shim in the exact call forms of the reference callers; outputs go back to
// Python for the oracle comparison.
// Usage: node tests/node/ops_gpu.js <dir>   (reads <dir>/manifest.json and <dir>/*.bin)
"use strict";

var fs = require("fs");
var path = require("path");

var sa = require(path.join(__dirname, "..", "..", "supra2-img-web_amd", "js", "index.js"));

var dir = process.argv[2];
var manifest = JSON.parse(fs.readFileSync(path.join(dir, "manifest.json"), "utf8"));

function loadBin(name, Type) {
  var b = fs.readFileSync(path.join(dir, name));
  var T = Type || Float32Array;
  return new T(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
}

function saveBin(name, arr) {
  fs.writeFileSync(path.join(dir, name), Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));
}

var forms = {
  // app/models/dit.js:169-173: one launch per sample on the packed qkv buffer
  dit_self_loop: function (gpu, c) {
    var D = 576, TOK = 256;
    var qkv = gpu.fromArray(loadBin(c.qkv), [c.B * TOK, 3 * D]);
    var a = gpu.empty([c.B * TOK, D]);
    for (var b = 0; b < c.B; b++) {
      var r = b * TOK * 3 * D;
      sa.attention(gpu, { q: qkv, k: qkv, v: qkv, Lq: TOK, Lk: TOK, H: 9, D: 64, ldq: 3 * D, ldk: 3 * D, ldv: 3 * D,
        qOff: r, kOff: r + D, vOff: r + 2 * D, oOff: b * TOK * D, out: a });
    }
    qkv.release();
    return a;
  },
  // the same batch in one launch with batch strides
  dit_self_batched: function (gpu, c) {
    var D = 576, TOK = 256;
    var qkv = gpu.fromArray(loadBin(c.qkv), [c.B * TOK, 3 * D]);
    var a = sa.attention(gpu, { B: c.B, q: qkv, k: qkv, v: qkv, Lq: TOK, Lk: TOK, H: 9, D: 64, ldq: 3 * D,
      ldk: 3 * D, ldv: 3 * D, kOff: D, vOff: 2 * D, sq: TOK * 3 * D, sk: TOK * 3 * D, sv: TOK * 3 * D,
      so: TOK * D });
    qkv.release();
    return a;
  },
  // app/models/dit.js:181-185: per-sample k|v buffers [L_b, 1152] at their true length
  dit_cross_loop: function (gpu, c) {
    var D = 576, TOK = 256;
    var q = gpu.fromArray(loadBin(c.q), [c.B * TOK, D]);
    var out = gpu.empty([c.B * TOK, D]);
    for (var b = 0; b < c.B; b++) {
      var kv = gpu.fromArray(loadBin(c.kv[b]), [c.L[b], 2 * D]);
      sa.attention(gpu, { q: q, k: kv, v: kv, Lq: TOK, Lk: c.L[b], H: 9, D: 64, ldq: D, ldk: 2 * D, ldv: 2 * D,
        qOff: b * TOK * D, kOff: 0, vOff: D, oOff: b * TOK * D, out: out });
      kv.release();
    }
    q.release();
    return out;
  },
  // the batched call-site helpers (js/dit_attn.js): one launch each for the whole batch
  dit_self_callsite: function (gpu, c) {
    var qkv = gpu.fromArray(loadBin(c.qkv), [c.B * 256, 3 * 576]);
    var a = sa.dit.selfAttention(gpu, qkv, c.B);
    qkv.release();
    return a;
  },
  dit_cross_callsite: function (gpu, c) {
    var q = gpu.fromArray(loadBin(c.q), [c.B * 256, 576]);
    var kvs = [];
    for (var b = 0; b < c.B; b++) kvs.push(gpu.fromArray(loadBin(c.kv[b]), [c.L[b], 2 * 576]));
    var ctx = sa.dit.packContexts(gpu, kvs, c.L);
    kvs.forEach(function (t) { t.release(); });
    var out = sa.dit.crossAttention(gpu, q, ctx);
    ctx.release();
    q.release();
    return out;
  },
  // app/gpu/ops.js:35-43 linear() in the DiT block forms (dit.js:167, 175, 191): W uploaded as
  // app/weights.js:89-101 does, gated or plain residual into an existing output
  linear: function (gpu, c) {
    var x = gpu.fromArray(loadBin(c.x), [c.M, c.K]);
    var W = { kind: "f32", N: c.N, K: c.K, buf: gpu.upload(loadBin(c.w)), bias: c.bias ? gpu.upload(loadBin(c.bias)) : null };
    var opts = { act: c.act };
    if (c.resid) {
      opts.out = gpu.fromArray(loadBin(c.y0), [c.M, c.N]);
      opts.resid = true;
    }
    if (c.gate) {
      opts.gate = gpu.fromArray(loadBin(c.gate), [c.gateLen]);
      opts.gOff = c.gOff;
    }
    var y = sa.linear(gpu, x, W, opts);
    x.release();
    if (opts.gate) opts.gate.release();
    gpu.native.free(W.buf);
    if (W.bias) gpu.native.free(W.bias);
    return y;
  },
  // app/models/vae.js:77-94 as one call: the weights as app/weights.js uploads them
  vae_block: function (gpu, c) {
    var C = c.C;
    var up = function (f) { return gpu.upload(loadBin(f)); };
    var lin = function (w, b) { return { kind: "f32", N: C, K: C, buf: up(w), bias: up(b) }; };
    var A = { norm: { g: up(c.gamma), b: up(c.beta) }, q: lin(c.wq, c.bq), k: lin(c.wk, c.bk), v: lin(c.wv, c.bv), o: lin(c.wo, c.bo) };
    var x = gpu.fromArray(loadBin(c.x), [c.HW, C]);
    var y = sa.vae.attention(gpu, x, c.HW, A);
    sa.vae.releaseWeights(gpu, A);
    return y;
  },
  // app/models/t5.js:73-80: dense [H, L, L] position bias, scale 1 (bias built on the device)
  t5_dense: function (gpu, c) {
    var q = gpu.fromArray(loadBin(c.q), [c.L, 768]);
    var k = gpu.fromArray(loadBin(c.k), [c.L, 768]);
    var v = gpu.fromArray(loadBin(c.v), [c.L, 768]);
    var bias = sa.positionBias(gpu, loadBin(c.table), 32, 12, c.L);
    var a = sa.attention(gpu, { q: q, k: k, v: v, Lq: c.L, Lk: c.L, H: 12, D: 64, ldq: 768, ldk: 768, ldv: 768,
      scale: 1, bias: bias });
    q.release(); k.release(); v.release(); bias.release();
    return a;
  },
  // the relative-position table gathered in-kernel plus a key-padding mask
  t5_relpos_mask: function (gpu, c) {
    var q = gpu.fromArray(loadBin(c.q), [c.L, 768]);
    var k = gpu.fromArray(loadBin(c.k), [c.L, 768]);
    var v = gpu.fromArray(loadBin(c.v), [c.L, 768]);
    var rp = sa.relposBias(gpu, loadBin(c.table), 32, 12, c.L, c.L);
    var km = gpu.fromArray(loadBin(c.mask, Uint8Array), [1, c.L]);
    var a = sa.attention(gpu, { q: q, k: k, v: v, Lq: c.L, Lk: c.L, H: 12, D: 64, ldq: 768, ldk: 768, ldv: 768,
      scale: 1, relpos: rp, keyMask: km });
    return a;
  },
  // app/models/dit.js:90 then dit.js:167: uploadLinear from a safetensors file feeding the linear layer
  st_linear: function (gpu, c) {
    return sa.weights.SafeTensors.open(c.file).then(function (st) {
      return sa.weights.uploadLinear(gpu, st, c.base).then(function (W) {
        var x = gpu.fromArray(loadBin(c.x), [c.M, W.K]);
        var y = sa.linear(gpu, x, W, {});
        x.release();
        gpu.native.free(W.buf);
        gpu.native.free(W.bias);
        st.close();
        return y;
      });
    });
  },
  // app/models/t5.js:72: embedding rows of the token ids, then gpu.fromArray
  st_rows: function (gpu, c) {
    return sa.weights.SafeTensors.open(c.file).then(function (st) {
      return st.rows(c.table, c.ids).then(function (rows) {
        st.close();
        return gpu.fromArray(rows, [c.ids.length, rows.length / c.ids.length]);
      });
    });
  },
  // app/models/vae.js:29: uploadConv3(gpu, st, "decoder.conv_in.", CIN_PAD)
  st_conv3: function (gpu, c) {
    return sa.weights.SafeTensors.open(c.file).then(function (st) {
      return sa.weights.uploadConv3(gpu, st, c.base, c.cinPad).then(function (W) {
        var out = gpu.empty([W.N * W.K]);
        gpu.native.copy(out.buf, 0, W.buf, 0, W.N * W.K * 4);
        gpu.sync();
        gpu.native.free(W.buf);
        if (W.bias) gpu.native.free(W.bias);
        st.close();
        return out;
      });
    });
  },
  // app/models/dit.js:72, 78-80: st.f32(name) on the host (here an F16 tensor), opened from bytes
  st_f32: function (gpu, c) {
    return sa.weights.SafeTensors.open(fs.readFileSync(c.file)).then(function (st) {
      return st.f32(c.tensor).then(function (a) {
        st.close();
        return gpu.fromArray(a);
      });
    });
  },
  // app/weights.js:28-37 on raw bytes: toF32(u8, "BF16") and bf16ToF32
  st_to_f32: function (gpu, c) {
    var u8 = new Uint8Array(loadBin(c.raw, Uint8Array));
    var a = sa.weights.toF32(u8, c.dtype);
    var b = sa.weights.bf16ToF32(u8);
    for (var i = 0; i < a.length; i++) {
      if (a[i] !== b[i] && !(a[i] !== a[i] && b[i] !== b[i])) throw new Error("bf16ToF32 != toF32 at " + i);
    }
    return gpu.fromArray(a);
  },
  // app/models/vae.js:86: single head, D = C = 512, default scale
  vae: function (gpu, c) {
    var q = gpu.fromArray(loadBin(c.q), [c.L, 512]);
    var k = gpu.fromArray(loadBin(c.k), [c.L, 512]);
    var v = gpu.fromArray(loadBin(c.v), [c.L, 512]);
    return sa.attention(gpu, { q: q, k: k, v: v, Lq: c.L, Lk: c.L, H: 1, D: 512, ldq: 512, ldk: 512, ldv: 512 });
  },
};

// The addon's buffer validation (what WebGPU checks for bindings and writeBuffer): every range a call
// touches must lie inside its buffer, released handles throw, overlapping copies are refused. Each
// of these throws before any device work, so nothing out of range reaches the GPU.
function boundaryChecks(gpu) {
  var n = gpu.native;
  var assert = require("assert");
  var code = function (c, re) {
    return function (e) { return e.code === c && re.test(e.message); };
  };
  var buf = n.malloc(256);
  var other = n.malloc(1024);
  n.upload(buf, new Float32Array(64), 0);                       // exactly fills it
  assert.throws(function () { n.upload(buf, new Float32Array(64), 4); }, code("SA_ERR_INVALID", /outside the 256-byte buffer/));
  assert.throws(function () { n.download(buf, new Float32Array(65), 0); }, code("SA_ERR_INVALID", /outside/));
  assert.throws(function () { n.memset(buf, 0, 257); }, code("SA_ERR_INVALID", /outside/));
  assert.throws(function () { n.copy(other, 0, buf, 128, 256); }, code("SA_ERR_INVALID", /copy src/));
  assert.throws(function () { n.copy(other, 0, other, 64, 128); }, code("SA_ERR_ALIAS", /overlap/));
  n.copy(other, 512, other, 0, 256);                            // disjoint ranges of one buffer are fine
  // Calls whose operand extent runs 8 bytes past its buffer (allocations are at least 256-byte
  // aligned, so the claimed range cannot reach another allocation and only the bounds check fires):
  // attention with q of 4 rows x 64 floats (1024 bytes) in a 1016-byte buffer
  var qb = n.malloc(1016), kv = n.malloc(1024), ob = n.malloc(1024);
  assert.throws(function () {
    n.attention({ B: 1, H: 1, D: 64, Lq: 4, Lk: 4, q: qb, k: kv, v: kv, out: ob, ldq: 64, ldk: 64, ldv: 64, scale: 1 });
  }, code("SA_ERR_INVALID", /^q: 1024 bytes at byte offset 0 lie outside the 1016-byte buffer/));
  // linear with y of 2 x 64 floats (512 bytes) in a 504-byte buffer, then x of 2 x 8 floats in 56 bytes
  var lx = n.malloc(64), lw = n.malloc(2048), ly = n.malloc(504), lx2 = n.malloc(56);
  assert.throws(function () { n.linear({ M: 2, N: 64, K: 8, x: lx, w: lw, y: ly }); },
    code("SA_ERR_INVALID", /^y: 512 bytes at byte offset 0 lie outside the 504-byte buffer/));
  assert.throws(function () { n.linear({ M: 2, N: 64, K: 8, x: lx2, w: lw, y: ob }); },
    code("SA_ERR_INVALID", /^x: 64 bytes at byte offset 0 lie outside the 56-byte buffer/));
  // a rejected call reports its own status, not a generic invalid-argument one
  assert.throws(function () {
    n.attention({ B: 1, H: 1, D: 64, Lq: 4, Lk: 4, q: kv, k: kv, v: kv, out: kv, ldq: 64, ldk: 64, ldv: 64, scale: 1 });
  }, code("SA_ERR_ALIAS", /output overlaps q, k or v/));
  assert.throws(function () {
    n.kernelName({ B: 1, H: 1, D: 2048, Lq: 1, Lk: 1, q: qb, k: qb, v: qb, out: ob, ldq: 2048, ldk: 2048, ldv: 2048,
                   scale: 1 });
  }, code("SA_ERR_UNSUPPORTED", /head dim 2048 exceeds/));
  [qb, kv, ob, lx, lw, ly, lx2].forEach(function (b) { n.free(b); });
  var ev = n.eventCreate();
  n.eventDestroy(ev);
  assert.throws(function () { n.eventRecord(ev); }, code("SA_ERR_INVALID", /has been released/));
  n.free(buf);
  assert.throws(function () { n.free(buf); }, code("SA_ERR_INVALID", /has been released/));
  assert.throws(function () { n.upload(buf, new Float32Array(4), 0); }, code("SA_ERR_INVALID", /has been released/));
  n.free(other);
  process.stdout.write("node: boundary checks passed\n");
}

sa.GPU.create().then(function (gpu) {
  boundaryChecks(gpu);
  var chain = Promise.resolve();
  manifest.cases.forEach(function (c) {
    chain = chain.then(function () {
      process.stdout.write("[node case] " + c.name + "\n");
      var out;
      return Promise.resolve(forms[c.form](gpu, c)).then(function (o) {
        out = o;
        return gpu.sync();
      }).then(function () {
        return gpu.read(out);
      }).then(function (data) {
        saveBin(c.name + ".out.bin", data);
        out.release();
      });
    });
  });
  return chain;
}).then(function () {
  process.stdout.write("node: all cases ran\n");
}, function (e) {
  process.stderr.write("node failure: " + (e.code || e.name) + ": " + e.message + "\n");
  process.exit(1);
});
