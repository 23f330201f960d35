"""The oracle's whole-model forward, prefill and sampler are bit-identical to
the reference engine's (oracle/_ref) on synthetic GGUF models: logits at
every step, every KV-cache byte, the RoPE tables and sampled tokens.

Each case runs in a subprocess because the reference keeps its model in
process globals.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from llama3pure_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    "llama_q8_0": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                       qtype=synth.Q8_0, seed=1),
    "llama_q4_0_tied": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=4, n_kv=4, vocab=512, ctx=128,
                            qtype=synth.Q4_0, seed=2, tied=True),
    "gemma_swa": dict(arch="gemma3", dim=256, hidden=768, n_layers=7, n_heads=4, n_kv=2, head_dim=64, vocab=512,
                      ctx=128, qtype=synth.Q8_0, seed=3, softcap=30.0, swa_window=12, norm_jitter=0.1, tied=True),
    # Q4_K with Q6_K down / V / output projections (a Q4_K_M-style mix)
    "llama_q4_k_m": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                         qtype=synth.Q4_K, seed=4, norm_jitter=0.1,
                         qtypes={"ffn_down": synth.Q6_K, "attn_v": synth.Q6_K, "output": synth.Q6_K}),
    # the other K-quants: Q5_K_M-, Q3_K_M- and Q2_K-style mixes
    "llama_q5_k_m": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                         qtype=synth.Q5_K, seed=5, norm_jitter=0.1,
                         qtypes={"ffn_down": synth.Q6_K, "attn_v": synth.Q6_K, "output": synth.Q6_K}),
    "llama_q3_k_m": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                         qtype=synth.Q3_K, seed=6, norm_jitter=0.1,
                         qtypes={"ffn_down": synth.Q4_K, "attn_v": synth.Q5_K, "output": synth.Q6_K}),
    "llama_q2_k": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                       qtype=synth.Q2_K, seed=7, norm_jitter=0.1,
                       qtypes={"ffn_down": synth.Q3_K, "attn_v": synth.Q3_K, "output": synth.Q6_K}),
    # the Q8_0-activation types (Q5_0 with Q5_1 V, Q4_1 down, IQ4_NL output
    # projection) and the half-precision types
    "llama_q5_0_mix": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                           qtype=synth.Q5_0, seed=8, norm_jitter=0.1,
                           qtypes={"output": synth.Q8_0, "attn_v": synth.Q5_1, "ffn_down": synth.Q4_1,
                                   "attn_output": synth.IQ4_NL}),   # later keys win ("output" is in "attn_output")
    "llama_f16_bf16": dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                           qtype=synth.F16, seed=9, norm_jitter=0.1,
                           qtypes={"ffn_down": synth.BF16, "attn_output": synth.BF16}),
    "gemma_bf16": dict(arch="gemma3", dim=256, hidden=768, n_layers=7, n_heads=4, n_kv=2, head_dim=64, vocab=512,
                       ctx=128, qtype=synth.BF16, seed=10, softcap=30.0, swa_window=12, norm_jitter=0.1, tied=True),
}


def run(tmp_path, kw, n_pre, n_dec, sample=None):
    if not oracle.have_ref():
        pytest.skip("oracle/_ref not built")
    p = tmp_path / "m.gguf"
    p.write_bytes(synth.synthetic_model(**kw))
    args = [sys.executable, os.path.join(HERE, "ref_model_check.py"), str(p), str(n_pre), str(n_dec), "7"]
    if sample:
        args += [str(v) for v in sample]
    out = subprocess.run(args, capture_output=True, text=True, timeout=600)
    i = out.stdout.rfind('{"ok"')     # the reference prints sampled tokens to stdout too
    assert i >= 0, out.stdout[-2000:] + out.stderr[-2000:]
    return json.loads(out.stdout[i:].splitlines()[0])


@pytest.mark.parametrize("name", list(CASES))
def test_forward_bit_identical(tmp_path, name):
    r = run(tmp_path, CASES[name], n_pre=40, n_dec=12)
    assert r["ok"], r
    assert r["kv_equal"] and r["rope_equal"], r


def test_sampler_bit_identical(tmp_path):
    r = run(tmp_path, CASES["llama_q8_0"], n_pre=8, n_dec=16, sample=(0.9, 40, 0.9))
    assert r["ok"], r
    assert len(set(r["sampled"])) > 1   # genuinely sampling, not argmax


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built (make -C oracle ref)")
def test_ref_drift_fixture_reproduces():
    """tests/golden/ref_drift.json is what the reference's -Ofast -fopenmp build gives now."""
    here = os.path.dirname(os.path.abspath(__file__))
    with open(os.path.join(here, "golden", "ref_drift.json")) as f:
        want = json.load(f)["models"]["llama_q8_0"]
    r = subprocess.run([sys.executable, os.path.join(here, "golden", "make_ref_drift.py"), "--one", "llama_q8_0"],
                       check=True, capture_output=True, text=True, timeout=600)
    got = json.loads(r.stdout.strip().splitlines()[-1])
    assert np.allclose(got["per_step"], want["per_step"], rtol=1e-6, atol=0)
