// Test helper: runs js/llama3pure.js as a Web Worker would see it and records
// what it posts.
//   node tests/js_shim_run.js <model.gguf> <scenarios.json>
// self.postMessage is a collector, so every message ("loaded", "token",
// "complete") is kept in order, next to the pieces cbRender receives and
// what console.error logs.  Each scenario is a "load" (with its options and a
// synthetic tokenizer) followed by a "generate":
//   {prompt: [ids], maxTokens, temperature, eos, eot, newline, seed, badModel}
// The tokenizer's encodeChat returns `prompt`; decode(id) is "\n" for
// `newline` and "<id>" otherwise.  Prints one JSON line: a list of
// {msgs, render, errors, ms} per scenario.
"use strict"
var fs = require("fs")
var path = require("path")

var messages = []
global.self = { postMessage: function (m) { messages.push(m) } }
var errors = []
console.error = function () {
  errors.push(Array.prototype.map.call(arguments, function (a) {
    return a && a.message ? a.message + " (code " + a.code + ")" : String(a)
  }).join(" "))
}
var llama3pure = require(path.join(__dirname, "..", "js", "llama3pure.js"))

var file = fs.readFileSync(process.argv[2])
var model = file.buffer.slice(file.byteOffset, file.byteOffset + file.length)
var scenarios = JSON.parse(fs.readFileSync(process.argv[3], "utf8"))
var results = []
scenarios.forEach(function (sc) {
  messages = []
  errors = []
  var render = []
  var tokenizer = {
    bosToken: 1,
    eosToken: sc.eos === undefined ? -1 : sc.eos,
    eotToken: sc.eot === undefined ? -1 : sc.eot,
    encodeChat: function (history, systemPrompt, isGemma) { return sc.prompt.slice() },
    decode: function (id) { return id === sc.newline ? "\n" : "<" + id + ">" },
  }
  var t0 = Date.now()
  llama3pure({
    type: "load",
    // badModel: the GGUF magic, version 9 and zeros
    model: sc.badModel ? new Uint8Array([0x47, 0x47, 0x55, 0x46, 9].concat(new Array(27).fill(0))).buffer : model,
    maxTokens: sc.maxTokens === undefined ? -1 : sc.maxTokens,
    temperature: sc.temperature === undefined ? 0.0 : sc.temperature,
    topK: 40,
    topP: 0.9,
    seed: sc.seed,
    tokenizer: tokenizer,
    cbRender: function (t) { render.push(t) },
  })
  llama3pure({ type: "generate", chatHistory: [{ role: "user", content: "hi" }] })
  results.push({ msgs: messages, render: render, errors: errors, ms: Date.now() - t0 })
})
llama3pure.close()
process.stdout.write(JSON.stringify(results) + "\n")
