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
    # Gemma with Q6_K V rows next to Q4_K Q and K rows: q, k and v run as three
    # GEMV launches, each applying the pending post-FFN norm to the residual
    "gemma_q4_k_m": dict(arch="gemma3", dim=512, hidden=1536, n_layers=4, n_heads=4, n_kv=2, head_dim=256,
                         vocab=2048, ctx=256, qtype=synth.Q4_K, seed=10, softcap=30.0, swa_window=16,
                         norm_jitter=0.1, tied=True, qtypes={"ffn_down": synth.Q6_K, "attn_v": synth.Q6_K}),
    "llama_q4_k_m": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                         qtype=synth.Q4_K, seed=4, norm_jitter=0.1,
                         qtypes={"ffn_down": synth.Q6_K, "attn_v": synth.Q6_K, "output": synth.Q6_K}),
    # Q4_K_M's per-layer mix: ffn_down Q6_K in layers 0 and 2 and Q4_K in
    # layers 1 and 3, so consecutive down GEMVs (each handing its sums of
    # squares to the next q|k|v) run different kernels and launch plans
    "llama_q4_k_m_alt": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048,
                             ctx=256, qtype=synth.Q4_K, seed=14, norm_jitter=0.1,
                             qtypes={"blk.0.ffn_down": synth.Q6_K, "blk.2.ffn_down": synth.Q6_K,
                                     "attn_v": synth.Q6_K, "output": synth.Q6_K}),
    # Q5_K_M-, Q3_K_M- and Q2_K-style mixes
    "llama_q5_k_m": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                         qtype=synth.Q5_K, seed=5, norm_jitter=0.1,
                         qtypes={"ffn_down": synth.Q6_K, "attn_v": synth.Q6_K, "output": synth.Q6_K}),
    "llama_q3_k_m": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                         qtype=synth.Q3_K, seed=6, norm_jitter=0.1,
                         qtypes={"ffn_down": synth.Q4_K, "attn_v": synth.Q5_K, "output": synth.Q6_K}),
    "llama_q2_k": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                       qtype=synth.Q2_K, seed=7, norm_jitter=0.1,
                       qtypes={"ffn_down": synth.Q3_K, "attn_v": synth.Q3_K, "output": synth.Q6_K}),
    # the Q8_0-activation types: Q5_0 with Q5_1 V, Q4_1 down, IQ4_NL output
    # projection (later keys win: "output" is also in "attn_output")
    "llama_q5_0_mix": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                           qtype=synth.Q5_0, seed=8, norm_jitter=0.1,
                           qtypes={"output": synth.Q8_0, "attn_v": synth.Q5_1, "ffn_down": synth.Q4_1,
                                   "attn_output": synth.IQ4_NL}),
    # half-precision weights: F16 with BF16 down and output projections
    "llama_f16_bf16": dict(arch="llama", dim=512, hidden=1024, n_layers=4, n_heads=8, n_kv=2, vocab=2048, ctx=256,
                           qtype=synth.F16, seed=9, norm_jitter=0.1,
                           qtypes={"ffn_down": synth.BF16, "attn_output": synth.BF16}),
}


_GEMMA = dict(arch="gemma3", head_dim=256, softcap=30.0, swa_window=16, tied=True)
_KMIX = {"ffn_down": synth.Q6_K, "attn_v": synth.Q6_K, "output": synth.Q6_K}

# One-layer models compared at position 0 (test_single_layer_position0_tight).
SINGLE_LAYER = {
    "llama_q8_0": dict(qtype=synth.Q8_0),
    "llama_q4_0": dict(qtype=synth.Q4_0),
    "gemma_q8_0": dict(qtype=synth.Q8_0, **_GEMMA),
    # Q4_K with Q6_K down / V / output projections, as in Q4_K_M files
    "llama_q4_k_m": dict(qtype=synth.Q4_K, qtypes=_KMIX),
    # rows that are not 16-byte multiples: Gemma-3-1B width 1152 (Q8_0 rows
    # of 1224 B), Gemma-3-270M width 640 (Q4_0 rows of 360 B), Q6_K at
    # widths 768 and 1280 (rows of 630 and 1050 B)
    "gemma_q8_0_1152": dict(qtype=synth.Q8_0, dim=1152, hidden=1536, n_heads=4, n_kv=1, **_GEMMA),
    # Gemma-2-2B widths (rows of 2304 and 9216 elements: short last chunk
    # columns), fused RMSNorm, GeGLU pair and post norms
    "gemma_q8_0_2304": dict(qtype=synth.Q8_0, dim=2304, hidden=9216, n_heads=8, n_kv=4, **_GEMMA),
    "llama_q4_0_640": dict(qtype=synth.Q4_0, dim=640, hidden=2048, n_heads=5, n_kv=1),
    "llama_q6_k_768": dict(qtype=synth.Q6_K, dim=768, hidden=1280, n_heads=6, n_kv=2),
    # every other weight type on its own, at widths that are not multiples of
    # a 2048-element chunk (and for Q4_1 / Q5_0 / Q5_1 / IQ4_NL / Q2_K / Q3_K,
    # rows that are not 16-byte multiples)
    "llama_q4_1_1120": dict(qtype=synth.Q4_1, dim=1120, hidden=1440, n_heads=5, n_kv=1),     # head size 224
    "llama_q5_0_1152": dict(qtype=synth.Q5_0, dim=1152, hidden=1536, n_heads=9, n_kv=3),
    "llama_q5_1_1120": dict(qtype=synth.Q5_1, dim=1120, hidden=1440, n_heads=5, n_kv=5),
    "llama_iq4_nl_640": dict(qtype=synth.IQ4_NL, dim=640, hidden=2048, n_heads=5, n_kv=1),
    "llama_q2_k_2304": dict(qtype=synth.Q2_K, dim=2304, hidden=1280, n_heads=18, n_kv=6),
    "llama_q3_k_2304": dict(qtype=synth.Q3_K, dim=2304, hidden=1280, n_heads=18, n_kv=6),
    "llama_q5_k_768": dict(qtype=synth.Q5_K, dim=768, hidden=1280, n_heads=6, n_kv=2),
    "llama_f16_640": dict(qtype=synth.F16, dim=640, hidden=1536, n_heads=5, n_kv=1),
    "llama_bf16_640": dict(qtype=synth.BF16, dim=640, hidden=1536, n_heads=5, n_kv=1),
    "llama_f32_640": dict(qtype=synth.F32, dim=640, hidden=1536, n_heads=5, n_kv=1),
}
SINGLE_TOKENS = (0, 7, 1234, 42, 555, 1000, 1999, 2047)


def single_layer_model(case):
    kw = dict(arch="llama", dim=512, hidden=1024, n_heads=8, n_kv=2)
    kw.update(SINGLE_LAYER[case])
    return synth.synthetic_model(n_layers=1, vocab=2048, ctx=64, seed=21, norm_jitter=0.1, **kw)


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


def kv_rows_diff(a, b, n_kv, seq_len, p0, p1):
    """|quant_a - quant_b| over the Q8_0 K or V cache blocks of positions [p0, p1)."""
    qa = a.reshape(n_kv, seq_len, -1, 34)[:, p0:p1, :, 2:].view(np.int8)
    qb = b.reshape(n_kv, seq_len, -1, 34)[:, p0:p1, :, 2:].view(np.int8)
    return np.abs(qa.astype(np.int32) - qb.astype(np.int32))


def _load_drift(key):
    p = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_drift.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f).get(key, {})


# name -> drift of the reference's -Ofast -fopenmp build from its plain build:
#   max_rel: max|dlogit|/rms(logits); kv["layer/k|v"]: max and mean |quant diff|
REF_DRIFT = _load_drift("models")
# single-layer case -> max|dlogit|/rms(logits) per token of SINGLE_TOKENS at position 0
SINGLE_DRIFT = _load_drift("single_layer")


# Long contexts against the oracle (tests/test_gpu_long_context.py): a prompt
# of `prompt` tokens through the batched prompt path (1024-row passes,
# attn_prefill_kernel), then teacher-forced decode steps whose attention spans
# the whole prompt (chunks + merge by default from 448 positions, from 192
# at head_dim >= 192; the per-head kernel forced for the later steps).  Small
# widths keep the oracle fast; the head shapes, GQA groups and windows are the
# ones the kernels specialise on.
LONG_CASES = {
    # head_dim 64, GQA 2, three prompt passes (2100 rows)
    "llama_hs64_2100": dict(model=dict(arch="llama", dim=256, hidden=512, n_layers=2, n_heads=4, n_kv=2, vocab=512,
                                       ctx=2304, qtype=synth.Q8_0, seed=51, norm_jitter=0.1), prompt=2100),
    # head_dim 128 (136-byte cache rows), GQA 4, two passes
    "llama_hs128_1100": dict(model=dict(arch="llama", dim=512, hidden=512, n_layers=2, n_heads=4, n_kv=1, vocab=512,
                                        ctx=1280, qtype=synth.Q8_0, seed=52, norm_jitter=0.1), prompt=1100),
    # Gemma head_dim 256 (32-position decode chunks), QK-norm, NEOX RoPE, a
    # 257-position window on five of six layers: windows start mid-prompt
    "gemma_hs256_swa_600": dict(model=dict(arch="gemma3", dim=512, hidden=512, n_layers=6, n_heads=2, n_kv=1,
                                           head_dim=256, vocab=512, ctx=768, qtype=synth.Q8_0, seed=53,
                                           softcap=30.0, swa_window=257, norm_jitter=0.1, tied=True), prompt=600),
    # Gemma head_dim 128, GQA 2, a 1000-position window at 2100 positions
    "gemma_hs128_swa_2100": dict(model=dict(arch="gemma3", dim=256, hidden=256, n_layers=6, n_heads=2, n_kv=1,
                                            head_dim=128, vocab=512, ctx=2304, qtype=synth.Q8_0, seed=54,
                                            softcap=30.0, swa_window=1000, norm_jitter=0.1, tied=True), prompt=2100),
    # 4300 positions: 68 decode chunks of 64, so the merge takes two rounds;
    # five prompt passes
    "llama_hs64_4300": dict(model=dict(arch="llama", dim=256, hidden=256, n_layers=2, n_heads=4, n_kv=2, vocab=512,
                                       ctx=4608, qtype=synth.Q8_0, seed=55, norm_jitter=0.1), prompt=4300),
}
LONG_STEPS = 4   # decode steps after the prompt (the last two on the per-head kernel)


def long_prompt(case):
    c = LONG_CASES[case]
    return np.random.default_rng(c["model"]["seed"] + 100).integers(0, c["model"]["vocab"], c["prompt"] + 1).astype(
        np.int32)


LONG_DRIFT = _load_drift("long")
