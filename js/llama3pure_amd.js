// llama3pure_amd.js — the JS engine's operator boundary on an MI355X.
//
// Drop-in for the three operations the reference's generate() calls
// (llama3pure-js-engine.js:7033-7183):
//   transformer(token, pos, computeLogits)         js:6121-6128 -> state.logits
//   transformerPrefill(allTokens, startPos, bs)    js:6130-6136
//   sample(logits, temp)                           js:6158-6267
// backed by libl3p through the N-API addon (l3p_napi.node).  Weights, KV
// cache and activations stay in HBM; transformer() copies the logits to the
// host only when computeLogits is set, as the reference fills state.logits
// only then.  decodeStep(token, pos) fuses forward and on-device sampling so
// only the token id crosses to JS.
//
// Sampling differs from the JS engine in one respect, by design: the JS
// engine draws from Math.random() (js:6141-6144), which nothing can
// reproduce; this backend draws from the C engine's xorshift64* generator
// (llama3pure-c-engine.c:4266-4276) with a settable seed.
"use strict"

var path = require("path")
var addon = require(path.join(__dirname, "l3p_napi.node"))

function Engine(device) {
  this.h = addon.open(device === undefined ? 0 : device)
  this.config = null
  this.logits = null
  this.topK = 40
  this.topP = 0.9
}

// loadModel (js:4288-4584): the GGUF bytes are parsed and uploaded once;
// the caller may drop the ArrayBuffer afterwards.  options: {swaPattern,
// attnSoftcap}, both optional and off by default (no counterpart in the
// reference: every swaPattern-th Gemma layer global instead of every 6th, and
// the attention score cap of Gemma-2).
Engine.prototype.load = function (model, contextSize, options) {
  this.config = addon.loadGguf(this.h, model, contextSize || 0, options || {})
  this.logits = null
  return this.config
}

Engine.prototype.transformer = function (token, pos, computeLogits) {
  if (computeLogits) {
    if (this.logits === null) {
      this.logits = new Float32Array(this.config.vocabSize)
    }
    addon.transformer(this.h, token, pos, true, this.logits)
  } else {
    addon.transformer(this.h, token, pos, false)
  }
}

Engine.prototype.transformerPrefill = function (allTokens, startPos, batchSize) {
  addon.transformerPrefill(this.h, allTokens, startPos, batchSize)
}

// sample(logits, temp): samples the logits of the last transformer() call,
// which are still on the device; `logits` is accepted for signature parity.
Engine.prototype.sample = function (logits, temp) {
  return addon.sample(this.h, temp, this.topK, this.topP)
}

Engine.prototype.decodeStep = function (token, pos, temp) {
  return addon.decode(this.h, token, pos, temp || 0.0, this.topK, this.topP)
}

Engine.prototype.setSeed = function (hi, lo) {
  addon.setSeed(this.h, hi >>> 0, lo >>> 0)
}

Engine.prototype.getSeed = function () {
  return addon.getSeed(this.h)
}

Engine.prototype.close = function () {
  addon.close(this.h)
}

module.exports = { Engine: Engine, addon: addon }
