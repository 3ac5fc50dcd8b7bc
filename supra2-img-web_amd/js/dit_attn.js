// Batched DiT attention call sites: one launch per block for self- and one for cross-attention.
//
// app/models/dit.js loops over its B samples and launches one attention per sample and block:
//   self  (dit.js:169-173): q, k, v are column blocks of the packed qkv [B*T, 3*dim] buffer, sample b
//         at row offset b*T;
//   cross (dit.js:180-185): sample b attends to its own prompt's k|v buffer [L_b, 2*dim]
//         (prepareContext, dit.js:137-144), k at column 0 and v at column dim.
// That is 2*B launches per block (128 for the batch-64 sweep). The helpers below issue one launch
// each for the whole batch through attention()'s batch strides; the cross-attention contexts are
// packed once per run into [B, Lmax, 2*dim] with per-sample key lengths (keys past L_b are masked,
// so the result equals the per-sample call at its true length).
//
//   selfAttention(gpu, qkv, B, opts)     -> Tensor [B*T, dim]
//   packContexts(gpu, kvs, lens, opts)   -> { kv, keyLen, lens, Lmax, B, release() }
//   crossAttention(gpu, q, ctx, opts)    -> Tensor [B*T, dim]
// opts: { tokens = 256, dim = 576, heads = 9, out } (the DiT config of app/models/dit.js).
"use strict";

var ops = require("./ops");

function cfg(opts) {
  var o = opts || {};
  var T = o.tokens === undefined ? 256 : o.tokens;
  var dim = o.dim === undefined ? 576 : o.dim;
  var H = o.heads === undefined ? 9 : o.heads;
  if (dim % H !== 0) throw new RangeError("dim must be a multiple of heads");
  return { T: T, dim: dim, H: H, D: dim / H, out: o.out };
}

// Self-attention of all B samples: equals the dit.js:169-173 loop.
function selfAttention(gpu, qkv, B, opts) {
  var c = cfg(opts);
  var ld = 3 * c.dim;
  return ops.attention(gpu, {
    B: B, q: qkv, k: qkv, v: qkv, Lq: c.T, Lk: c.T, H: c.H, D: c.D, ldq: ld, ldk: ld, ldv: ld,
    qOff: 0, kOff: c.dim, vOff: 2 * c.dim, sq: c.T * ld, sk: c.T * ld, sv: c.T * ld, so: c.T * c.dim, out: c.out,
  });
}

// Packs per-sample k|v tensors kvs[b] ([lens[b], 2*dim], rows contiguous) into one [B*Lmax, 2*dim]
// tensor (device-to-device copies, stream-ordered) plus an int32 key-length tensor. Rows past
// lens[b] are left unwritten: the kernel never reads keys at or past a sequence's length.
function packContexts(gpu, kvs, lens, opts) {
  var c = cfg(opts);
  var B = kvs.length;
  if (lens.length !== B) throw new RangeError("one length per context");
  var Lmax = 1;
  for (var b = 0; b < B; b++) {
    if (!(lens[b] >= 0)) throw new RangeError("context lengths must be >= 0");
    Lmax = Math.max(Lmax, lens[b]);
  }
  var row = 2 * c.dim * 4;  // bytes per k|v row
  var kv = gpu.empty([B * Lmax, 2 * c.dim]);
  for (b = 0; b < B; b++) {
    if (lens[b] === 0) continue;
    if (!kvs[b] || !kvs[b].buf) {
      var e = new Error("context " + b + " is a released or invalid Tensor");
      e.code = "SA_ERR_INVALID";
      throw e;
    }
    gpu.op({ name: "copy", flops: 0 }, function () {
      gpu.native.copy(kv.buf, b * Lmax * row, kvs[b].buf, 0, lens[b] * row);
    });
  }
  var hostLens = Int32Array.from(lens);
  var keyLen = gpu.fromArray(hostLens, [B]);
  return {
    kv: kv, keyLen: keyLen, lens: hostLens, Lmax: Lmax, B: B,
    release: function () { kv.release(); keyLen.release(); },
  };
}

// Cross-attention of all B samples to their packed contexts: equals the dit.js:180-185 loop.
function crossAttention(gpu, q, ctx, opts) {
  var c = cfg(opts);
  var ldkv = 2 * c.dim;
  return ops.attention(gpu, {
    B: ctx.B, q: q, k: ctx.kv, v: ctx.kv, Lq: c.T, Lk: ctx.Lmax, H: c.H, D: c.D, ldq: c.dim, ldk: ldkv, ldv: ldkv,
    qOff: 0, kOff: 0, vOff: c.dim, sq: c.T * c.dim, sk: ctx.Lmax * ldkv, sv: ctx.Lmax * ldkv, so: c.T * c.dim,
    // host lengths: the flash kernel's balanced schedule, or short sequences packed in small launches
    keyLen: ctx.keyLen, keyLenHost: ctx.lens, out: c.out,
  });
}

module.exports = { selfAttention: selfAttention, packContexts: packContexts, crossAttention: crossAttention };
