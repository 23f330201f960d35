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
    # Q4_K_M's per-layer mix: ffn_down Q6_K in layers 0 and 2, Q4_K in 1 and 3
    "llama_q4_k_m_alt": dict(arch="llama", dim=256, hidden=512, n_layers=4, n_heads=8, n_kv=2, vocab=512, ctx=128,
                             qtype=synth.Q4_K, seed=14, norm_jitter=0.1,
                             qtypes={"blk.0.ffn_down": synth.Q6_K, "blk.2.ffn_down": synth.Q6_K,
                                     "attn_v": synth.Q6_K, "output": synth.Q6_K}),
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


def test_attention_options_refused_out_of_range(cpuref):
    """The oracle's set_attention takes the library's option ranges: negative
    swa_pattern or attn_softcap, an infinite cap (inf * tanh(s / inf) is NaN)
    and a NaN cap are refused; 0 and finite caps are taken."""
    m = cpuref.open_model(synth.synthetic_model(**CASES["gemma_swa"]))
    try:
        for pat, cap in ((-1, 0.0), (2, -1.0), (2, float("inf")), (2, float("nan"))):
            with pytest.raises(ValueError):
                m.set_attention(pat, cap)
        m.set_attention(2, 50.0)
        m.set_attention(0, 0.0)
    finally:
        m.close()


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


def _gemma_layers(rng, dim, hidden, qd, kvd):
    w = lambda r, c: rng.normal(0, 0.05, (r, c)).astype(np.float32)
    return {"attn_q": w(qd, dim), "attn_k": w(kvd, dim), "attn_v": w(kvd, dim), "attn_output": w(dim, qd),
            "ffn_gate": w(hidden, dim), "ffn_up": w(hidden, dim), "ffn_down": w(dim, hidden)}


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built (make -C oracle ref)")
@pytest.mark.parametrize("pattern,n_layers", [(2, 2), (3, 3), (2, 4)])
def test_swa_pattern_option_against_reference(tmp_path, pattern, n_layers):
    """The oracle's swa_pattern option (no counterpart in the reference, which
    hard-codes every 6th layer global, c:5100) pinned against the reference
    itself.  A Gemma layer whose matrices are all zero leaves the residual
    bit-identical (its projections, post norms and GeGLU are all zero), so the
    reference on a model with zero layers inserted where its fixed pattern
    puts sliding-window layers runs the same computation as the oracle with
    pattern p on the model without them: layers l with l % p < p - 1 local,
    the others global with the global RoPE base.  Logits at every decode step
    bit-identical, and the K/V caches of the mapped layers byte-identical."""
    if not oracle.have_ref():
        pytest.skip("oracle/_ref not built")
    dim, hidden, heads, kv, hd, vocab = 128, 256, 2, 1, 64, 256
    rng = np.random.default_rng(60 + 10 * pattern + n_layers)
    layers = [_gemma_layers(rng, dim, hidden, heads * hd, kv * hd) for _ in range(n_layers)]
    emb = rng.normal(0, 0.5, (vocab, dim)).astype(np.float32)
    # reference layer of each oracle layer: the oracle's local layers fill
    # the reference's local slots (l % 6 < 5) and its global layers the
    # reference's global slots (l % 6 == 5), in order
    ref_of, rl = [], 0
    for l in range(n_layers):
        glob = l % pattern == pattern - 1
        while (rl % 6 == 5) != glob:
            rl += 1
        ref_of.append(rl)
        rl += 1
    n_ref = ref_of[-1] + 1
    zero = {k: np.zeros_like(v) for k, v in layers[0].items()}

    def model(n, at):
        mats = {"token_embd.weight": emb}
        for l in range(n):
            src = layers[at.index(l)] if l in at else zero
            mats.update({f"blk.{l}.{k}.weight": v for k, v in src.items()})
        return synth.synthetic_model(arch="gemma3", dim=dim, hidden=hidden, n_layers=n, n_heads=heads, n_kv=kv,
                                     head_dim=hd, vocab=vocab, ctx=64, qtype=synth.Q8_0, seed=0, tied=True,
                                     softcap=30.0, swa_window=5, rope_theta=1e6, rope_theta_swa=1e4, mats=mats)

    pr, po = tmp_path / "ref.gguf", tmp_path / "orc.gguf"
    pr.write_bytes(model(n_ref, ref_of))
    po.write_bytes(model(n_layers, list(range(n_layers))))
    out = subprocess.run([sys.executable, os.path.join(HERE, "ref_swa_check.py"), str(pr), str(po), str(pattern),
                          "20", "8", ",".join(map(str, ref_of))], capture_output=True, text=True, timeout=600)
    i = out.stdout.rfind('{"ok"')
    assert i >= 0, out.stdout[-2000:] + out.stderr[-2000:]
    r = json.loads(out.stdout[i:].splitlines()[0])
    assert r["ok"] and r["steps"] == 8 and r["kv_equal"], r
