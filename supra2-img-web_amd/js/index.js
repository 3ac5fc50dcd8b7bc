// Entry point of the JS binding: the device runtime, the attention operator and the batched DiT
// call sites.
"use strict";

var device = require("./device");
var ops = require("./ops");
var dit = require("./dit_attn");

module.exports = {
  GPU: device.GPU,
  Tensor: device.Tensor,
  BufferPool: device.BufferPool,
  attention: ops.attention,
  attentionKernel: ops.attentionKernel,
  relativeBucket: ops.relativeBucket,
  relposBias: ops.relposBias,
  positionBias: ops.positionBias,
  dit: dit,
};
