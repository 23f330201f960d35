// llama3pure.js — the JS engine's public entry point, llama3pure(data)
// (llama3pure-js-engine.js:7185-7260), and its generation loop
// (js:7033-7183), run on an MI355X through llama3pure_amd.js and libl3p.
//
// Messages, options and stop rules are the reference's:
//   llama3pure({type: "load", model: ArrayBuffer, maxTokens, contextSize,
//               systemPrompt, temperature, topP, topK, cbRender, ...})
//       loads the GGUF into HBM and posts {type: "loaded"};
//   llama3pure({type: "generate", chatHistory})
//       posts {type: "token", token: text} for each piece of decoded text
//       (cbRender(text) receives the same pieces, in the same order), then
//       {type: "complete", output: all text}.
// Messages go to self.postMessage when the file runs as a Web Worker (it then
// also listens on self.onmessage), as the reference's do.  Generation stops
// at the end-of-sequence or end-of-turn token (not emitted), when the
// absolute position reaches maxTokens (<= 0 or above the context: the
// context), or when, on a step divisible by 10 with more than 20 tokens
// generated, the last 10 tokens equal each of at least 6 windows of 10 right
// before them.  A decoded "\n" is held back and emitted only before the next
// piece of text, so a newline just before the end is dropped.  Errors are
// caught and logged with console.error.
//
// What differs from the reference, by design:
//   * the tokenizer is injected with the "load" message (data.tokenizer):
//       encodeChat(chatHistory, systemPrompt, isGemma) -> array of token ids
//       decode(id) -> text of the token (a Llama tokenizer may hold back
//                     bytes of an incomplete UTF-8 sequence)
//       flush() -> text held back at the end (optional)
//       bosToken, eosToken, eotToken
//     The BPE tokenizer and chat templates stay on the host, outside the
//     forward path this backend replaces;
//   * the prompt, all but its last token, is prefilled with one call:
//     libl3p takes 1024 positions per pass over the weights where the
//     reference takes PREFILL_BATCH_SIZE = 32 (js:3159); the KV cache holds
//     the same rows either way;
//   * each generated token is one decodeStep: the forward step and the
//     sampler run on the device and only the token id comes back to JS;
//   * sampling draws from the C engine's xorshift64* generator
//     (llama3pure-c-engine.c:4266-4276), seeded by data.seed ([hi, lo]
//     uint32 words) when given, where the reference calls Math.random();
//   * two optional load fields the reference lacks, data.swaPattern (every
//     swaPattern-th Gemma layer global instead of every 6th) and
//     data.attnSoftcap (Gemma-2's attention score cap), off when absent.
"use strict"

var path = require("path")
var Engine = require(path.join(__dirname, "llama3pure_amd.js")).Engine

// options, with the reference's defaults (js:218-223)
var opt = {
  temperature: 0.9,
  topP: 0.9,
  topK: 40,
  systemPrompt: "You are a helpful assistant.",
  maxTokens: -1,
  contextSize: 0,
}
var cbRender = null
var tokenizer = null
var engine = null
var config = null

function inWorker() {
  return typeof self !== "undefined" && typeof self.postMessage === "function"
}

function post(msg) {
  if (inWorker()) {
    self.postMessage(msg)
  }
  if (msg.type === "token" && cbRender) {
    cbRender(msg.token)
  }
}

// The last 10 tokens of g repeat in at least 6 consecutive windows of 10
// directly before them (up to 10 windows are looked at).
function repeating(g) {
  var n = g.length
  var runs = 0
  for (var w = 1; w <= 10; w++) {
    var start = n - 10 - 10 * w
    if (start < 0) {
      break
    }
    for (var i = 0; i < 10; i++) {
      if (g[start + i] !== g[n - 10 + i]) {
        return runs > 5
      }
    }
    runs++
  }
  return runs > 5
}

function load(data) {
  var keys = ["maxTokens", "contextSize", "systemPrompt", "temperature", "topP", "topK"]
  for (var i = 0; i < keys.length; i++) {
    if (data[keys[i]] !== undefined) {
      opt[keys[i]] = data[keys[i]]
    }
  }
  if (typeof data.cbRender === "function") {
    cbRender = data.cbRender
  }
  if (data.tokenizer !== undefined) {
    tokenizer = data.tokenizer
  }
  if (!(data.model instanceof ArrayBuffer)) {
    console.error("The model parameter is required and must be an ArrayBuffer.")
    return
  }
  if (engine === null) {
    engine = new Engine(0)
  }
  config = null
  config = engine.load(new Uint8Array(data.model), opt.contextSize,
                       { swaPattern: data.swaPattern, attnSoftcap: data.attnSoftcap })
  if (Array.isArray(data.seed)) {
    engine.setSeed(data.seed[0], data.seed[1])
  }
  post({ type: "loaded" })
}

function generate(chatHistory) {
  if (!tokenizer) {
    throw new Error("no tokenizer: pass data.tokenizer with the load message")
  }
  engine.topK = opt.topK
  engine.topP = opt.topP
  var prompt = tokenizer.encodeChat(chatHistory, opt.systemPrompt, config.isGemma)
  if (!prompt || prompt.length === 0) {
    prompt = [tokenizer.bosToken]
  }
  var n = prompt.length
  var last = opt.maxTokens
  if (last <= 0 || last > config.seqLen) {
    last = config.seqLen
  }
  var pos = 0
  if (n > 1) {
    engine.transformerPrefill(Int32Array.from(prompt), 0, n - 1)
    pos = n - 1
  }
  var token = prompt[pos]
  var output = ""
  var held = false   // a decoded "\n" not yet emitted
  var generated = []
  // every step here is at a position >= n - 1, where the reference computes
  // logits and samples (js:7085-7093)
  for (; pos < last; pos++) {
    var next = engine.decodeStep(token, pos, opt.temperature)
    if (next === tokenizer.eosToken || next === tokenizer.eotToken) {
      break
    }
    generated.push(next)
    var text = tokenizer.decode(next)
    if (text === "\n") {
      held = true
    } else {
      if (held) {
        output += "\n"
        post({ type: "token", token: "\n" })
        held = false
      }
      if (text.length > 0) {
        output += text
        post({ type: "token", token: text })
      }
      if (generated.length > 20 && pos % 10 === 0 && repeating(generated)) {
        break
      }
    }
    token = next
  }
  if (typeof tokenizer.flush === "function") {
    var rest = tokenizer.flush()
    if (rest && rest.length > 0) {
      output += rest
      post({ type: "token", token: rest })
    }
  }
  post({ type: "complete", output: output })
  return output
}

function llama3pure(data) {
  try {
    if (data.type === "load") {
      load(data)
    } else if (data.type === "generate") {
      if (config !== null) {
        generate(data.chatHistory)
      }
    }
  } catch (err) {
    console.error(err)
  }
}

// Not in the reference: releases the device context (the process exit does too).
llama3pure.close = function () {
  if (engine !== null) {
    engine.close()
    engine = null
    config = null
  }
}

if (inWorker()) {
  self.onmessage = function (e) {
    llama3pure(e.data)
  }
}

module.exports = llama3pure
