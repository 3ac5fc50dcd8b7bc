// The attention operator for the Supra2-Img Web callers, on MI355X.
//
// attention(gpu, opts) keeps the surface of app/gpu/ops.js:103-149, so the four call sites
// (app/models/dit.js:172, dit.js:184, t5.js:80, vae.js:86) work unchanged:
//   q: [Lq, ldq] with head h at column qOff + h*D; k, v: [Lk, ldk] / [Lk, ldv] at kOff / vOff + h*D;
//   output rows [Lq, H*D] written at element offset oOff of `out` (allocated when omitted);
//   scale defaults to 1/sqrt(D); bias: additive [H, Lq, Lk] score bias (a Tensor).
// Every call is one launch of the fused kernel, whatever the head dim or bias (the reference's
// unfused chunked path and its "must fit in one chunk" limit do not exist here).
//
// Additive options (absent in the reference, defaults keep its behaviour):
//   B, sq, sk, sv, so  batch of B sequences in one launch (element strides between sequences),
//                      which folds the per-sample loops of dit.js:170-185 into one call;
//   ldo                output row stride (default H*D, as ops.js:114);
//   keyLen             Tensor int32 [B]: keys j >= keyLen[b] are masked (padded cross-attention);
//   keyLenHost         optional Int32Array copy of keyLen on the host: the library then balances
//                      the sequences over the CUs (results come from keyLen either way);
//   keyMask, smask     Tensor uint8 [B, smask]: nonzero = attend (SDPA boolean convention);
//   relpos             { table: Tensor f32 [numBuckets, H], lut: Tensor i32 [Lq + Lk - 1] }: the
//                      T5 relative-position bias gathered in-kernel instead of a dense bias;
//   sbias              batch stride of a dense bias (default 0: shared).
// A query row with no attended key yields zeros.
"use strict";

function handle(t, name) {
  if (t === undefined || t === null) return null;
  if (!t.buf) {
    var e = new Error(name + " is a released or invalid Tensor");
    e.code = "SA_ERR_INVALID";
    throw e;
  }
  return t.buf;
}

function def(x, d) {
  return x === undefined || x === null ? d : x;
}

// ops.attention arguments -> the addon's sa_attn_args object.
function nativeArgs(o, out) {
  var H = o.H;
  var D = o.D;
  var args = {
    B: def(o.B, 1),
    H: H,
    D: D,
    Lq: o.Lq,
    Lk: o.Lk,
    q: handle(o.q, "q"),
    k: handle(o.k, "k"),
    v: handle(o.v, "v"),
    out: handle(out, "out"),
    qOff: def(o.qOff, 0),
    kOff: def(o.kOff, 0),
    vOff: def(o.vOff, 0),
    oOff: def(o.oOff, 0),
    ldq: o.ldq,
    ldk: o.ldk,
    ldv: o.ldv,
    ldo: def(o.ldo, H * D),
    sq: def(o.sq, 0),
    sk: def(o.sk, 0),
    sv: def(o.sv, 0),
    so: def(o.so, def(o.ldo, H * D) * o.Lq),
    scale: def(o.scale, 1 / Math.sqrt(D)),
    biasMode: 0,
    maskMode: 0,
  };
  if (o.relpos) {
    args.biasMode = 2;
    args.bias = handle(o.relpos.table, "relpos.table");
    args.bucketLut = handle(o.relpos.lut, "relpos.lut");
    args.numBuckets = o.relpos.table.shape[0];
  } else if (o.bias) {
    args.biasMode = 1;
    args.bias = handle(o.bias, "bias");
    args.sbias = def(o.sbias, 0);
  }
  if (o.keyLen) {
    args.maskMode = 1;
    args.keyLen = handle(o.keyLen, "keyLen");
    if (o.keyLenHost) args.keyLenHost = o.keyLenHost;
  } else if (o.keyMask) {
    args.maskMode = 2;
    args.keyMask = handle(o.keyMask, "keyMask");
    args.smask = def(o.smask, o.Lk);
  }
  return args;
}

// Profiler flops of a call as the reference counts them (app/gpu/ops.js:116: 4*Lq*Lk*D*H, where a
// caller passes each sample its own key count), summed over the B sequences: a key-length call
// counts each sequence's attended keys, min(max(keyLen[b], 0), Lk), when their host copy came along
// (keyLenHost); without it the padded Lk (the device lengths are not read back for a count).
function attentionFlops(o) {
  var B = def(o.B, 1);
  var keys = B * o.Lk;
  if (o.keyLen && o.keyLenHost) {
    keys = 0;
    for (var b = 0; b < B; b++) keys += Math.min(Math.max(o.keyLenHost[b] | 0, 0), o.Lk);
  }
  return 4 * o.Lq * keys * o.D * o.H;
}

function attention(gpu, o) {
  var B = def(o.B, 1);
  var out = o.out || gpu.empty([B * o.Lq, o.H * o.D]);
  var args = nativeArgs(o, out);
  // device scratch for the calls that merge partial results across workgroups (wide heads), from
  // the pool and released right away: the pool hands buffers out again in queue order
  var wsBytes = gpu.native.workspaceBytes(args);
  var ws = null;
  if (wsBytes > 0) {
    ws = gpu.empty([Math.ceil(wsBytes / 4)]);
    args.workspace = ws.buf;
    args.workspaceBytes = wsBytes;
  }
  try {
    gpu.op({ name: "attention", flops: attentionFlops(o) }, function () {
      gpu.native.attention(args);
    });
  } finally {
    if (ws) ws.release();
  }
  return out;
}

// Name of the kernel a call would launch (validation and selection only, no launch).
function attentionKernel(gpu, o) {
  var out = o.out || gpu.empty([def(o.B, 1) * o.Lq, o.H * o.D]);
  try {
    return gpu.native.kernelName(nativeArgs(o, out));
  } finally {
    if (out !== o.out) out.release();
  }
}

// HF T5 relative-position bucket of rel = j - i (app/models/t5.js:14-23), float32 arithmetic.
function relativeBucket(rel, buckets, maxDistance, native) {
  var nat = native || require("./device").loadNative();
  var nb = def(buckets, 32);
  var md = def(maxDistance, 128);
  // one LUT entry: Lq = 1 - min(rel, 0) puts rel at a valid index
  var Lq = rel < 0 ? 1 - rel : 1;
  var Lk = rel > 0 ? rel + 1 : 1;
  return nat.bucketLut(Lq, Lk, nb, md, true)[rel + Lq - 1];
}

// Device tensors for the in-kernel relative-position bias of an [Lq, Lk] attention:
// { table: [numBuckets, H] (the checkpoint's relative_attention_bias), lut: bucket of j - i }.
function relposBias(gpu, table, numBuckets, H, Lq, Lk, maxDistance) {
  var lut = gpu.native.bucketLut(Lq, Lk, numBuckets, def(maxDistance, 128), true);
  return {
    table: table instanceof Float32Array ? gpu.fromArray(table, [numBuckets, H]) : table,
    lut: gpu.fromArray(lut, [Lq + Lk - 1]),
  };
}

// Dense [H, L, L] bias on the device, the tensor app/models/t5.js:55-65 builds on the CPU and
// uploads per prompt (t5.js:73); for callers that keep passing `bias`.
function positionBias(gpu, table, numBuckets, H, L, maxDistance) {
  var rp = relposBias(gpu, table, numBuckets, H, L, L, maxDistance);
  var out = gpu.empty([H, L, L]);
  gpu.op({ name: "positionBias", flops: 0 }, function () {
    gpu.native.positionBias(rp.table.buf, rp.lut.buf, numBuckets, H, L, L, out.buf);
  });
  if (rp.table !== table) rp.table.release();
  rp.lut.release();
  return out;
}

module.exports = {
  attention: attention,
  attentionKernel: attentionKernel,
  nativeArgs: nativeArgs,
  relativeBucket: relativeBucket,
  relposBias: relposBias,
  positionBias: positionBias,
};
