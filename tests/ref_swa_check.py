"""Subprocess helper for test_oracle_model.py: the reference engine
(oracle/_ref/libref.so) on one GGUF and the oracle on another, with the
oracle's sliding-window pattern set, fed the same tokens; compares the logits
of every decode step bit for bit and the K/V caches of mapped layers.

usage: python tests/ref_swa_check.py <ref.gguf> <oracle.gguf> <swa_pattern> <n_prefill> <n_decode> <map>
map: comma-separated reference layer for each oracle layer.  Prints one JSON line.
"""
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import oracle  # noqa: E402


def main():
    ref_path, orc_path = sys.argv[1], sys.argv[2]
    pattern, n_pre, n_dec = int(sys.argv[3]), int(sys.argv[4]), int(sys.argv[5])
    layer_map = [int(v) for v in sys.argv[6].split(",")]
    ref = oracle.Ref()
    rc = ref.lib.ref_model_open(ref_path.encode(), 0)
    if rc != 0:
        print(json.dumps({"ok": False, "why": f"ref_model_open rc={rc}"}))
        return
    cr = oracle.CpuRef()
    m = cr.open_model(open(orc_path, "rb").read(), 0)
    m.set_attention(pattern, 0.0)
    toks = np.random.default_rng(11).integers(0, m.vocab, n_pre + 1).astype(np.int32)
    res = {"ok": True, "steps": 0, "kv_equal": True}
    pos = 0
    while pos < n_pre:
        bs = min(32, n_pre - pos)
        ref.lib.ref_prefill(oracle._vp(toks), pos, bs)
        m.prefill(toks, pos, bs)
        pos += bs
    tok = int(toks[n_pre])
    out_r = np.empty(m.vocab, np.float32)
    for step in range(n_dec):
        ref.lib.ref_forward(tok, pos, 1, oracle._vp(out_r))
        lo = m.forward(tok, pos)
        if not np.array_equal(lo, out_r):
            res.update(ok=False, why=f"logits differ at step {step}", maxdiff=float(np.abs(lo - out_r).max()))
            break
        tok = int(np.argmax(lo))
        pos += 1
        res["steps"] = step + 1
    for layer, rl in enumerate(layer_map):
        for wv in (0, 1):
            n = m.kv(layer, wv).size
            a = np.empty(n, np.uint8)
            ref.lib.ref_copy_kv(rl, wv, oracle._vp(a), n)
            if not np.array_equal(a, m.kv(layer, wv)):
                res["kv_equal"] = False
    print(json.dumps(res))


if __name__ == "__main__":
    main()
