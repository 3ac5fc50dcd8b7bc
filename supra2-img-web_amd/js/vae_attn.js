// The SD-VAE mid-block attention as one call: attention(gpu, x, hw, A) does what
// VAEDecoder.attention (app/models/vae.js:77-94) does with four ops and ten launches,
//   n = groupnorm(x, A.norm.g, A.norm.b, C, 32, no SiLU); q, k, v = linear(n, A.q / A.k / A.v);
//   a = attention(q, k, v, one head of dim C); out = x + linear(a, A.o),
// through sa_vae_attention_f32 (GroupNorm, one q|k|v projection, the attention kernels, the output
// projection with the residual fused). A holds the weights as app/weights.js uploads them
// ({ kind, N, K, buf, bias } per linear, norm.g / norm.b device buffers); the q, k and v weights
// are packed once into one [3C, C] buffer (and [3C] bias) on the device and cached on A.
// As in the reference, x is consumed: the result is written over x, which is returned.
"use strict";

function raw(t) {
  if (t === undefined || t === null) return null;
  return typeof t === "object" && "buf" in t && "shape" in t ? t.buf : t;
}

function invalid(msg) {
  var e = new Error(msg);
  e.code = "SA_ERR_INVALID";
  return e;
}

// [3C, C] weight and [3C] bias from A.q, A.k, A.v (device-to-device copies, stream-ordered)
function packQkv(gpu, A, C) {
  if (A._saQkv) return A._saQkv;
  var parts = [A.q, A.k, A.v];
  parts.forEach(function (W) {
    if (!W || W.N !== C || W.K !== C) throw invalid("q, k, v weights must be [C, C] with C = " + C);
  });
  var hasBias = parts.every(function (W) { return !!W.bias; });
  if (!hasBias && parts.some(function (W) { return !!W.bias; })) {
    throw invalid("q, k and v must all have biases or none");
  }
  var wq = gpu.native.malloc(3 * C * C * 4);
  var bq = hasBias ? gpu.native.malloc(3 * C * 4) : null;
  parts.forEach(function (W, i) {
    gpu.native.copy(wq, i * C * C * 4, raw(W.buf), 0, C * C * 4);
    if (bq) gpu.native.copy(bq, i * C * 4, raw(W.bias), 0, C * 4);
  });
  A._saQkv = { w: wq, b: bq };
  return A._saQkv;
}

function attention(gpu, x, hw, A, opts) {
  var o = opts || {};
  var C = x.shape[1];
  if (!x.buf) throw invalid("x is a released or invalid Tensor");
  var qkv = packQkv(gpu, A, C);
  var args = {
    HW: hw, C: C, groups: o.groups || 32, eps: o.eps === undefined ? 1e-6 : o.eps,
    x: x.buf, gamma: raw(A.norm.g), beta: raw(A.norm.b), wqkv: qkv.w, bqkv: qkv.b,
    wo: raw(A.o.buf), bo: raw(A.o.bias), out: x.buf,
  };
  var bytes = gpu.native.vaeWorkspaceBytes(args);
  var ws = gpu.empty([Math.ceil(bytes / 4)]);
  args.workspace = ws.buf;
  args.workspaceBytes = bytes;
  try {
    // q|k|v and output projections plus the attention (4 * HW^2 * C)
    var flops = 2 * hw * 3 * C * C + 4 * hw * hw * C + 2 * hw * C * C;
    gpu.op({ name: "vaeAttention", flops: flops }, function () {
      gpu.native.vaeAttention(args);
    });
  } finally {
    ws.release();  // stream-ordered pool reuse
  }
  return x;
}

// Frees the packed q|k|v weights cached on A.
function releaseWeights(gpu, A) {
  if (!A._saQkv) return;
  gpu.native.free(A._saQkv.w);
  if (A._saQkv.b) gpu.native.free(A._saQkv.b);
  A._saQkv = null;
}

module.exports = { attention: attention, releaseWeights: releaseWeights };
