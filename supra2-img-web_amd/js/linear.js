// The linear layer for the Supra2-Img Web callers, on MI355X: linear(gpu, x, W, opts) keeps the
// surface of app/gpu/ops.js:33-43,
//   y = x @ W^T (+ bias) (act);  opts.out + opts.resid: out += (gate[gOff + n] *) y, in place;
//   opts.rows / opts.aOff: use `rows` rows of x starting at element offset aOff;
// with W = { kind: "f32", N, K, buf, bias } as app/weights.js:89-101 uploads it ([N, K], PyTorch
// layout; buf and bias are device buffers from gpu.upload or Tensors). act is "none", "gelu",
// "gelu_tanh" or "silu" (app/gpu/gemm.js:21-36). One launch of sa_linear_f32 per call.
"use strict";

var ACT = { none: 0, gelu: 1, gelu_tanh: 2, silu: 3 };

function invalid(msg) {
  var e = new Error(msg);
  e.code = "SA_ERR_INVALID";
  return e;
}

// Tensor -> its device buffer; a raw device buffer passes through; null/undefined -> null.
function raw(t, name) {
  if (t === undefined || t === null) return null;
  if (typeof t === "object" && "buf" in t && "shape" in t) {
    if (!t.buf) throw invalid(name + " is a released or invalid Tensor");
    return t.buf;
  }
  return t;
}

function linear(gpu, x, W, opts) {
  var o = opts || {};
  if (W.kind !== undefined && W.kind !== "f32") throw invalid("only f32 weights are supported (W.kind = " + W.kind + ")");
  var M = o.rows !== undefined && o.rows !== null ? o.rows : x.size / W.K;
  if (!(M >= 1) || Math.floor(M) !== M) throw invalid("rows must be a positive integer (x.size / W.K = " + M + ")");
  var act = ACT[o.act === undefined || o.act === null ? "none" : o.act];
  if (act === undefined) throw invalid("unknown act " + o.act);
  var out = o.out || gpu.empty([M, W.N]);
  var args = {
    M: M,
    N: W.N,
    K: W.K,
    x: raw(x, "x"),
    xOff: o.aOff || 0,
    w: raw(W.buf, "W.buf"),
    bias: raw(o.bias || W.bias, "bias"),
    act: act,
    epilogue: o.resid ? (o.gate ? 2 : 1) : 0,
    gate: o.resid && o.gate ? raw(o.gate, "gate") : null,
    gateOff: o.gOff || 0,
    y: raw(out, "out"),
  };
  // flops 2*M*N*K, the reference's matmul meta (app/gpu/ops.js:15-31)
  gpu.op({ name: "linear", flops: 2 * M * W.N * W.K }, function () {
    gpu.native.linear(args);
  });
  return out;
}

// Name of the kernel a call would launch (validation and selection only, no launch).
function linearKernel(gpu, x, W, opts) {
  var o = opts || {};
  var M = o.rows !== undefined && o.rows !== null ? o.rows : x.size / W.K;
  var out = o.out || gpu.empty([M, W.N]);
  try {
    return gpu.native.linearKernelName({
      M: M, N: W.N, K: W.K, x: raw(x, "x"), xOff: o.aOff || 0, w: raw(W.buf, "W.buf"),
      bias: raw(o.bias || W.bias, "bias"), act: ACT[o.act || "none"], epilogue: o.resid ? (o.gate ? 2 : 1) : 0,
      gate: o.resid && o.gate ? raw(o.gate, "gate") : null, gateOff: o.gOff || 0, y: raw(out, "out"),
    });
  } finally {
    if (out !== o.out) out.release();
  }
}

module.exports = { linear: linear, linearKernel: linearKernel, ACT: ACT };
