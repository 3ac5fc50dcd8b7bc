// Entry point of the JS binding: the device runtime, the attention operator, the batched DiT call
// sites, the linear layer either side of attention, the VAE mid-block attention and the
// safetensors weight loader.
"use strict";

var device = require("./device");
var ops = require("./ops");
var dit = require("./dit_attn");
var lin = require("./linear");
var vae = require("./vae_attn");
var weights = require("./weights");

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
  linear: lin.linear,
  linearKernel: lin.linearKernel,
  vae: vae,
  weights: weights,
};
