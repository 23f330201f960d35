"""Long contexts against the oracle: prompts of 600 to 4300 tokens through the
batched prompt path, then decode steps attending over the whole prompt.

Covered paths: attn_prefill_kernel over 1024-row prompt passes (two to five
passes), the decode chunk + merge kernels (including the second merge round
past 64 chunks at 4300 positions and the 32-position chunks of head_dim 256),
the per-head decode kernel at the same lengths, sliding windows that start in
the middle of the prompt, head_dim 64, 128 and 256, GQA groups of 2 and 4.

Tolerances (the same policy as the short full-model tests), per case from
tests/golden/ref_drift.json "long" (the reference's -Ofast -fopenmp build
against its plain build on the same protocol):
  * K/V cache of every layer over every written position: quants within
    max(1, drift max + 1), mean difference within max(1%, 3 * drift mean);
  * logits per step: max|dlogit| <= max(1e-2, 2 * drift) * rms(logits);
  * argmax identical unless the oracle's top-2 margin is within 2 * tolerance.
Every case prints its worst ratio to each bound.
"""
import numpy as np
import pytest

import llama3pure_amd as l3p
from llama3pure_amd import synth
from model_cases import LONG_CASES, LONG_DRIFT, LONG_STEPS, kv_quant_diff, long_prompt, rms

pytestmark = pytest.mark.gpu


def margin(lo):
    s = np.sort(lo)
    return float(s[-1] - s[-2])


@pytest.mark.parametrize("case", list(LONG_CASES))
def test_long_context_against_oracle(torch_gpu, cpuref, monkeypatch, case):
    c = LONG_CASES[case]
    P = c["prompt"]
    drift = LONG_DRIFT[case]
    g = synth.synthetic_model(**c["model"])
    toks = long_prompt(case)
    with l3p.Context(0) as ctx:
        ctx.load_gguf(g)
        m = cpuref.open_model(g)
        try:
            ctx.prefill(toks[:P], 0)
            m.prefill(toks, 0, P)
            # the prompt's K/V rows, every layer
            kv_ratio = 0.0
            for layer in range(m.n_layers):
                for wv in (False, True):
                    d = kv_quant_diff(ctx.copy_kv(layer, wv), m.kv(layer, wv), m, P)
                    r = drift["kv"][f"{layer}/{'v' if wv else 'k'}"]
                    lim_max, lim_mean = max(1, r["max"] + 1), max(0.01, 3.0 * r["mean"])
                    kv_ratio = max(kv_ratio, float(d.mean()) / lim_mean)
                    assert d.max() <= lim_max and d.mean() <= lim_mean, \
                        (case, layer, wv, int(d.max()), float(d.mean()), lim_max, lim_mean)
            # decode steps over the whole prompt: chunks + merge, then per-head
            tok, pos = int(toks[P]), P
            lo_ratio = 0.0
            tol_rel = max(1e-2, 2.0 * drift["max_rel"])
            for step in range(LONG_STEPS):
                monkeypatch.setenv("L3P_ATTN_HEAD", "1" if step >= LONG_STEPS // 2 else "0")
                lo_ref = m.forward(tok, pos)
                lo_gpu = ctx.forward(tok, pos)
                tol = tol_rel * rms(lo_ref)
                err = float(np.max(np.abs(lo_gpu - lo_ref)))
                lo_ratio = max(lo_ratio, err / tol)
                assert err <= tol, f"{case} step {step} (pos {pos}): max |dlogit| {err:.3g} > {tol:.3g}"
                if margin(lo_ref) > 2 * tol:
                    assert int(np.argmax(lo_gpu)) == int(np.argmax(lo_ref)), (case, step)
                tok, pos = int(np.argmax(lo_ref)), pos + 1
            monkeypatch.delenv("L3P_ATTN_HEAD", raising=False)
            # the decode steps' own K/V rows as well
            for layer in range(m.n_layers):
                for wv in (False, True):
                    d = kv_quant_diff(ctx.copy_kv(layer, wv), m.kv(layer, wv), m, pos)
                    assert d.max() <= max(1, drift["kv"][f"{layer}/{'v' if wv else 'k'}"]["max"] + 1), \
                        (case, layer, wv, "after decode")
            print(f"[long] {case}: {P} prompt positions + {LONG_STEPS} steps; worst logit err/tol {lo_ratio:.3f}, "
                  f"worst KV mean-flip/limit {kv_ratio:.3f}", flush=True)
        finally:
            m.close()
