"""Subprocess helper for test_oracle_model.py: runs the reference engine
(oracle/_ref/libref.so, which keeps its model in process globals) and the
oracle on one synthetic GGUF, and reports the first difference.

usage: python tests/ref_model_check.py <model.gguf> <n_prefill> <n_decode> <seed> [temp topk topp]
Prints one JSON line.
"""
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import oracle  # noqa: E402


def main():
    path, n_pre, n_dec, seed = sys.argv[1], int(sys.argv[2]), int(sys.argv[3]), int(sys.argv[4])
    sample = None if len(sys.argv) < 8 else (float(sys.argv[5]), int(sys.argv[6]), float(sys.argv[7]))
    ref = oracle.Ref()
    rc = ref.lib.ref_model_open(path.encode(), 0)
    if rc != 0:
        print(json.dumps({"ok": False, "why": f"ref_model_open rc={rc}"}))
        return
    cr = oracle.CpuRef()
    m = cr.open_model(open(path, "rb").read(), 0)
    rng = np.random.default_rng(seed)
    toks = rng.integers(0, m.vocab, n_pre + 1).astype(np.int32)
    res = {"ok": True, "steps": 0, "kv_equal": True, "rope_equal": True, "sampled": []}
    # rope tables
    half = m.head_dim // 2
    for swa in ((0, 1) if m.is_gemma else (0,)):
        for p in (0, 1, 5, m.seq_len - 1):
            c, s = np.empty(half, np.float32), np.empty(half, np.float32)
            ref.lib.ref_rope_row(swa, p, oracle._vp(c), oracle._vp(s))
            oc, os_ = m.rope_row(bool(swa), p)
            if not (np.array_equal(c.view(np.uint32), oc.view(np.uint32)) and
                    np.array_equal(s.view(np.uint32), os_.view(np.uint32))):
                res["rope_equal"] = False
    # prefill in the reference's batches of 32 (c:5277-5287) on both sides
    pos = 0
    while pos < n_pre:
        bs = min(32, n_pre - pos)
        ref.lib.ref_prefill(oracle._vp(toks), pos, bs)
        m.prefill(toks, pos, bs)
        pos += bs
    tok = int(toks[n_pre])
    out_r = np.empty(m.vocab, np.float32)
    st = 0x2545F4914F6CDD1D
    for step in range(n_dec):
        if sample is None:
            ref.lib.ref_forward(tok, pos, 1, oracle._vp(out_r))
            lo = m.forward(tok, pos)
            if not np.array_equal(lo.view(np.uint32), out_r.view(np.uint32)):
                res.update(ok=False, why=f"logits differ at step {step}", maxdiff=float(np.abs(lo - out_r).max()))
                break
            tok = int(np.argmax(lo))
        else:
            t, p, k = sample[0], sample[2], sample[1]
            s = C_ull(st)
            nxt = ref.lib.ref_generate_token(tok, pos, t, k, p, s)
            lo = m.forward(tok, pos)
            mine, st2 = cr.sample(lo, t, k, p, st)
            res["sampled"].append(int(nxt))
            if mine != nxt or st2 != s.value:
                res.update(ok=False, why=f"sample differs at step {step}: {mine} vs {nxt}")
                break
            st = s.value
            tok = int(nxt)
        pos += 1
        res["steps"] = step + 1
    for layer in range(m.n_layers):
        for wv in (0, 1):
            n = m.kv(layer, wv).size
            a = np.empty(n, np.uint8)
            ref.lib.ref_copy_kv(layer, wv, oracle._vp(a), n)
            if not np.array_equal(a, m.kv(layer, wv)):
                res["kv_equal"] = False
    print(json.dumps(res))


def C_ull(v):
    import ctypes
    return ctypes.c_ulonglong(v)


if __name__ == "__main__":
    import ctypes
    # ref_generate_token takes a pointer; wrap byref at call sites
    _orig = oracle.Ref.__init__

    def _init(self, *a, **k):
        _orig(self, *a, **k)
        f = self.lib.ref_generate_token
        self.lib.ref_generate_token = lambda tok, pos, t, k2, p, s: f(tok, pos, t, k2, p, ctypes.byref(s))
    oracle.Ref.__init__ = _init
    main()
