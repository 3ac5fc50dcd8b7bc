// Entry point of the JS binding: the device runtime and the attention operator.
"use strict";

var device = require("./device");
var ops = require("./ops");

module.exports = {
  GPU: device.GPU,
  Tensor: device.Tensor,
  BufferPool: device.BufferPool,
  attention: ops.attention,
  attentionKernel: ops.attentionKernel,
  relativeBucket: ops.relativeBucket,
  relposBias: ops.relposBias,
  positionBias: ops.positionBias,
};
