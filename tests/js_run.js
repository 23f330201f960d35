// Test helper: drives the JS boundary (js/llama3pure_amd.js) the way the
// reference's generate() drives its engine (llama3pure-js-engine.js:7033-7183)
// and writes what it saw.
//   node tests/js_run.js <model.gguf> <out.bin> <prompt ids comma-separated> <steps> [swaPattern attnSoftcap]
// Prefill in batches of 32 (PREFILL_BATCH_SIZE), then `steps` greedy steps
// with transformer(..., true) + sample(state.logits, 0).  out.bin holds, per
// step, the vocab logits (float32) followed by the sampled id (int32).
"use strict"
var fs = require("fs")
var path = require("path")
var m = require(path.join(__dirname, "..", "js", "llama3pure_amd.js"))

var model = fs.readFileSync(process.argv[2])
var prompt = process.argv[4].split(",").map(Number)
var steps = Number(process.argv[5])
var eng = new m.Engine(0)
var opts = process.argv.length > 7 ? { swaPattern: Number(process.argv[6]), attnSoftcap: Number(process.argv[7]) } : undefined
var cfg = eng.load(new Uint8Array(model.buffer, model.byteOffset, model.length), 0, opts)
var pos = 0
var prefillEnd = prompt.length - 1
while (pos < prefillEnd) {
  var bs = Math.min(32, prefillEnd - pos)
  eng.transformerPrefill(prompt, pos, bs)
  pos += bs
}
var token = prompt[pos]
var out = Buffer.alloc(steps * (cfg.vocabSize * 4 + 4))
var off = 0
for (var s = 0; s < steps; s++) {
  eng.transformer(token, pos, true)
  var next = eng.sample(eng.logits, 0.0)
  Buffer.from(eng.logits.buffer).copy(out, off)
  off += cfg.vocabSize * 4
  out.writeInt32LE(next, off)
  off += 4
  token = next
  pos += 1
}
fs.writeFileSync(process.argv[3], out)
eng.close()
console.log(JSON.stringify({ ok: true, steps: steps, vocab: cfg.vocabSize, isGemma: cfg.isGemma,
                            swaPattern: cfg.swaPattern, attnSoftcap: cfg.attnSoftcap }))
