"""Synthetic models shared by the GPU model tests and the fixture script
tests/golden/make_ref_drift.py."""
import json
import os

import numpy as np

from llama3pure_amd import synth

MODELS = {
    "llama_q8_0": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                       qtype=synth.Q8_0, seed=1, norm_jitter=0.1),
    "llama_q4_0": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                       qtype=synth.Q4_0, seed=2, tied=True, norm_jitter=0.1),
    "gemma_q8_0": dict(arch="gemma3", dim=512, hidden=1536, n_layers=7, n_heads=4, n_kv=2, head_dim=256,
                       vocab=2048, ctx=256, qtype=synth.Q8_0, seed=3, softcap=30.0, swa_window=16,
                       norm_jitter=0.1, tied=True),
}


def rms(lo):
    return float(np.sqrt(np.mean(lo.astype(np.float64) ** 2)))


def teacher_prompt(m):
    """The 20-token prompt of the teacher-forced protocol."""
    return np.random.default_rng(11).integers(0, m.vocab, 20).astype(np.int32)


def kv_quant_diff(a, b, m, pos):
    """|quant_a - quant_b| over the Q8_0 K or V cache blocks of positions [0, pos)."""
    qa = a.reshape(m.n_kv, m.seq_len, -1)[:, :pos].reshape(m.n_kv, pos, -1, 34)[..., 2:].view(np.int8)
    qb = b.reshape(m.n_kv, m.seq_len, -1)[:, :pos].reshape(m.n_kv, pos, -1, 34)[..., 2:].view(np.int8)
    return np.abs(qa.astype(np.int32) - qb.astype(np.int32))


def _load_drift():
    p = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_drift.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f)["models"]


# name -> drift of the reference's -Ofast -fopenmp build from its plain build:
#   max_rel: max|dlogit|/rms(logits); kv["layer/k|v"]: max and mean |quant diff|
REF_DRIFT = _load_drift()
