"""Subprocess helper for tests/test_gpu_full_configs.py: runs the reference
engine's optimised build (oracle/_ref/libref_omp.so, its Makefile's
-Ofast -fopenmp line) on one GGUF file so a test can measure how far the
reference drifts from its own plain build (the oracle) on exactly the
protocol the test applies to the GPU.  One model per process: the reference
keeps its model in process globals.

usage: python tests/ref_drift_run.py <job.json>

job keys:
  gguf        path of the model file
  prompt      path of an int32 .npy of prompt tokens; the first n_prompt are
              prefilled in the reference's batches of 32 (c:5277-5287)
  n_prompt
  kv_out      .npy written after the prompt: uint8 [n_layers, 2, layer bytes]
              (K then V of every layer, the cache layout c:365-372)
  kv_in       optional .npy of the same shape installed after the prompt
  steps       optional int32 .npy [n, 2] of (token, position) decode steps,
              run teacher-forced with logits
  logits_out  .npy float32 [n, vocab] of those steps' logits
  kv_end_out  optional .npy of the whole cache after the steps
"""
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import oracle  # noqa: E402


def dump_kv(ref, n_layers, layer_bytes):
    out = np.empty((n_layers, 2, layer_bytes), np.uint8)
    for layer in range(n_layers):
        for wv in (0, 1):
            ref.lib.ref_copy_kv(layer, wv, oracle._vp(out[layer, wv]), layer_bytes)
    return out


def main():
    with open(sys.argv[1]) as f:
        job = json.load(f)
    ref = oracle.Ref(oracle.REF_OMP_SO)
    rc = ref.lib.ref_model_open(job["gguf"].encode(), 0)
    if rc != 0:
        raise SystemExit(f"ref_model_open rc={rc}")
    info = job["info"]   # n_layers, layer_bytes, vocab
    toks = np.ascontiguousarray(np.load(job["prompt"]), np.int32)
    pos = 0
    while pos < job["n_prompt"]:
        bs = min(32, job["n_prompt"] - pos)
        ref.lib.ref_prefill(oracle._vp(toks), pos, bs)
        pos += bs
    np.save(job["kv_out"], dump_kv(ref, info["n_layers"], info["layer_bytes"]))
    print("prompt done", flush=True)
    if job.get("kv_in"):
        kv = np.load(job["kv_in"])
        for layer in range(info["n_layers"]):
            for wv in (0, 1):
                src = np.ascontiguousarray(kv[layer, wv])
                if ref.lib.ref_set_kv(layer, wv, oracle._vp(src), src.size) != 0:
                    raise SystemExit("ref_set_kv failed")
    if job.get("steps"):
        steps = np.load(job["steps"])
        lo = np.empty((len(steps), info["vocab"]), np.float32)
        for i, (tok, p) in enumerate(steps):
            ref.lib.ref_forward(int(tok), int(p), 1, oracle._vp(lo[i]))
        np.save(job["logits_out"], lo)
        if job.get("kv_end_out"):
            np.save(job["kv_end_out"], dump_kv(ref, info["n_layers"], info["layer_bytes"]))
    print("ok", flush=True)


if __name__ == "__main__":
    main()
