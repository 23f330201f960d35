"""The benchmark workloads at full architecture against the oracle.

Both build the exact model and prompt that bench.py times (weights drawn
N(0, 0.02) on the GPU with the bench's seeds and quantized to Q8_0 by the
library's quantizer); the oracle reads the same GGUF image.

* Llama-3-8B architecture, greedy decode from KV position 1024 (the bench's
  headline): 32 layers, dim 4096, 32/8 heads of 128, SwiGLU 14336, vocab
  128256, theta 5e5, 2048-position context.
    - The first 32 prompt positions go through both prompt paths (the GPU's
      MFMA GEMM and attn_prefill_kernel, the oracle's transformer_prefill
      restatement); the K/V caches of all 32 layers are compared.
    - The GPU then prefills the bench's 1024-token prompt and its whole K/V
      cache is installed in the oracle (the prompt path at long range is
      pinned by test_gpu_long_context.py; the oracle would need minutes for
      1024 full-size positions), so both decode from the same state.
    - Free-running: l3p_generate_greedy (the call the bench times) decodes
      128 steps from position 1024 on the GPU, the oracle runs its own greedy
      loop from the same cache; the token sequences must be identical, and a
      divergence is accepted only at a step whose oracle top-2 margin is
      within twice the logits tolerance (a near-tie).
    - Teacher-forced: the GPU decodes the same 128 steps fed the oracle's
      tokens; its logits are held to the tolerance at every step, its argmax
      may differ from the oracle's only at near-ties and at no more than
      twice as many steps as the reference's own -Ofast build flips on the
      same steps, plus two; the decode steps' K/V rows are compared.
* Gemma-2-2B architecture (26 layers, dim 2304, 8/4 heads of 256, GeGLU
  9216, vocab 256000, tied embedding, final soft-cap 30): both sides run the
  bench's 511-position prompt, then the workload's 128 decode steps sampled
  at temperature 0.9, top-k 40, top-p 0.9 from xorshift64* seed 42, both
  sides fed the oracle's token each step.  At every step the RNG states are
  identical and the device sampler's token is exactly the reference
  sampler's on the GPU's own logits.  A sampled token flips wherever the
  draw lands within the logits' difference of a CDF boundary, which at these
  depths happens between the reference's own two builds too: the count of
  steps whose token differs from the oracle's is held to twice the count the
  reference's -Ofast build shows on the same steps, plus two.  Two tests:
    - the reference's gemma3 semantics (every 6th layer global, no
      attention cap), which the reference's own builds run, so the drift is
      measured on exactly this protocol;
    - the workload as benched: alternating local/global layers and attention
      soft-cap 50 (the load options swa_pattern=2 and attn_softcap=50, the
      oracle's set_attention(2, 50)), held to the tolerances the first
      protocol measured, since the reference cannot run these options.

Tolerances: the full-model policy, with the drift measured on the same model
and protocol by running the reference's own -Ofast -fopenmp build
(tests/ref_drift_run.py) beside the oracle (its plain build, bit for bit):
  * K/V quants within max(1, drift max + 1) of the oracle's, mean difference
    within max(1%, 3 * drift mean), per layer.  Through 32 layers the
    reference's two builds already differ in several percent of the deep
    layers' quants: Q8_0 requantization of Q, K and V at every layer turns
    last-bit differences into one-step flips that grow with depth;
  * logits per step within max(1e-2, 2 * drift) * rms(logits), drift the
    largest max|dlogit|/rms of the reference's builds over the steps;
  * greedy tokens identical unless the oracle's top-2 margin is within twice
    the tolerance.
Each test prints its worst ratio to each bound.
"""
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np
import pytest

import bench
import llama3pure_amd as l3p
from llama3pure_amd import synth
from model_cases import kv_rows_diff, rms

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
C4_DECODE_STEPS = 128     # the workload's 128 decode steps: positions 1024..1151
C5_DECODE_STEPS = 128     # the workload's 128 sampled steps


def margin(lo):
    s = np.sort(lo)
    return float(s[-1] - s[-2])


def log(msg):
    print(f"[full] {msg}", flush=True)


def all_kv(get, n_layers):
    """[n_layers, 2, layer bytes]: K then V of every layer from get(layer, which_v)."""
    return np.stack([np.stack([get(layer, False), get(layer, True)]) for layer in range(n_layers)])


def run_reference(img, info, prompt, n_prompt, kv_in=None, steps=None):
    """The reference's -Ofast -fopenmp build on the same model: its K/V cache
    after the prompt, and (with steps) the logits of teacher-forced decode
    steps from the installed cache kv_in and its cache after them."""
    import oracle
    if not os.path.exists(oracle.REF_OMP_SO):
        pytest.skip("oracle/_ref/libref_omp.so not built")
    d = tempfile.mkdtemp(dir="/dev/shm" if os.path.isdir("/dev/shm") else None)
    try:
        job = {"gguf": os.path.join(d, "m.gguf"), "prompt": os.path.join(d, "prompt.npy"), "n_prompt": n_prompt,
               "kv_out": os.path.join(d, "kv.npy"), "info": info}
        img.tofile(job["gguf"])
        np.save(job["prompt"], prompt)
        if kv_in is not None:
            job["kv_in"] = os.path.join(d, "kv_in.npy")
            np.save(job["kv_in"], kv_in)
        if steps is not None:
            job.update(steps=os.path.join(d, "steps.npy"), logits_out=os.path.join(d, "logits.npy"),
                       kv_end_out=os.path.join(d, "kv_end.npy"))
            np.save(job["steps"], np.asarray(steps, np.int32))
        with open(os.path.join(d, "job.json"), "w") as f:
            json.dump(job, f)
        r = subprocess.run([sys.executable, os.path.join(HERE, "ref_drift_run.py"), os.path.join(d, "job.json")],
                           capture_output=True, text=True, timeout=900)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
        out = {"kv": np.load(job["kv_out"])}
        if steps is not None:
            out["logits"] = np.load(job["logits_out"])
            out["kv_end"] = np.load(job["kv_end_out"])
        return out
    finally:
        shutil.rmtree(d, ignore_errors=True)


def kv_bounds(ref_kv, orc_kv, n_kv, seq_len, p0, p1):
    """Per layer and K/V: the (max, mean) quant-difference limits from the
    reference builds' own difference over positions [p0, p1)."""
    lims = []
    for layer in range(ref_kv.shape[0]):
        row = []
        for wv in (0, 1):
            d = kv_rows_diff(ref_kv[layer, wv], orc_kv[layer, wv], n_kv, seq_len, p0, p1)
            row.append((max(1, int(d.max()) + 1), max(0.01, 3.0 * float(d.mean())), float(d.mean())))
        lims.append(row)
    return lims


def check_kv(gpu_kv, orc_kv, lims, n_kv, seq_len, p0, p1, what):
    worst, worst_ref = 0.0, 0.0
    for layer in range(gpu_kv.shape[0]):
        for wv in (0, 1):
            d = kv_rows_diff(gpu_kv[layer, wv], orc_kv[layer, wv], n_kv, seq_len, p0, p1)
            lmax, lmean, rmean = lims[layer][wv]
            worst = max(worst, float(d.mean()) / lmean)
            worst_ref = max(worst_ref, rmean)
            assert d.max() <= lmax and d.mean() <= lmean, (what, layer, wv, int(d.max()), float(d.mean()), lmax, lmean)
    return worst, worst_ref


def test_llama3_8b_greedy_decode_from_1024(torch_gpu, cpuref):
    t0 = time.perf_counter()
    with l3p.Context(0) as ctx:
        img = synth.synthetic_model(qtype=synth.Q8_0, make_mat=synth.gpu_q8_0_maker(ctx, torch_gpu, 99),
                                    **bench.LLAMA3_8B)
        mi = ctx.load_gguf(img)
        m = cpuref.open_model(img)
        try:
            L, nkv, S = mi.n_layers, mi.n_kv_heads, mi.seq_len
            prompt = np.random.default_rng(5).integers(0, mi.vocab_size, 1025).astype(np.int32)
            log(f"llama3-8b: model {img.nbytes / 1e9:.2f} GB built and loaded ({time.perf_counter() - t0:.1f} s)")
            # the prompt paths on the first 32 positions
            ctx.prefill(prompt[:32], 0)
            m.prefill(prompt, 0, 32)
            gpu_kv32 = all_kv(ctx.copy_kv, L)
            orc_kv32 = all_kv(m.kv, L)
            # the bench's 1024-position prompt on the GPU, its cache into the oracle
            ctx.prefill(prompt[:1024], 0)
            kv1024 = all_kv(ctx.copy_kv, L)
            for layer in range(L):
                for wv in (0, 1):
                    m.set_kv(layer, bool(wv), kv1024[layer, wv])
            log(f"llama3-8b: prompts done, decoding ({time.perf_counter() - t0:.1f} s)")
            # free-running greedy: the benched call on the GPU, the oracle's own loop
            free_gpu = ctx.generate_greedy(int(prompt[1024]), 1024, C4_DECODE_STEPS)
            assert len(free_gpu) == C4_DECODE_STEPS
            tok, pos = int(prompt[1024]), 1024
            steps, lo_rs, free_orc, margins = [], [], [], []
            for step in range(C4_DECODE_STEPS):
                steps.append((tok, pos))
                lo_r = m.forward(tok, pos)
                lo_rs.append(lo_r)
                margins.append(margin(lo_r) / rms(lo_r))
                tok, pos = int(np.argmax(lo_r)), pos + 1
                free_orc.append(tok)
            diverge = next((i for i in range(C4_DECODE_STEPS) if free_gpu[i] != free_orc[i]), None)
            # teacher-forced: the GPU decodes the oracle's steps (the oracle's
            # side of them is its free run above)
            errs, mism = [], []
            for step, (tok, pos_i) in enumerate(steps):
                tok_g, _ = ctx.decode(tok, pos_i, temperature=0.0)
                lo_g = ctx.logits()
                assert tok_g == int(np.argmax(lo_g)), f"step {step}: device argmax is not the first maximum"
                errs.append(float(np.max(np.abs(lo_g - lo_rs[step]))) / rms(lo_rs[step]))
                if tok_g != free_orc[step]:
                    mism.append(step)
            gpu_end, orc_end = all_kv(ctx.copy_kv, L), all_kv(m.kv, L)
            log(f"llama3-8b: {len(steps)} decode steps, reference build running ({time.perf_counter() - t0:.1f} s)")
            ref = run_reference(img, {"n_layers": L, "layer_bytes": int(gpu_kv32.shape[2]), "vocab": mi.vocab_size},
                                prompt, 32, kv_in=kv1024, steps=steps)
            # bounds from the reference's own builds
            kv_lims = kv_bounds(ref["kv"], orc_kv32, nkv, S, 0, 32)
            drift = max(float(np.max(np.abs(ref["logits"][i] - lo))) / rms(lo) for i, lo in enumerate(lo_rs))
            tol_rel = max(1e-2, 2.0 * drift)
            ref_flips = [i for i in range(len(steps)) if int(np.argmax(ref["logits"][i])) != free_orc[i]]
            kv_w, kv_ref = check_kv(gpu_kv32, orc_kv32, kv_lims, nkv, S, 0, 32, "prompt")
            worst = max(errs) / tol_rel
            near = max((margins[s] for s in mism), default=0.0) / (2 * tol_rel)
            log(f"llama3-8b: free-running greedy through l3p_generate_greedy, positions 1024-{1023 + C4_DECODE_STEPS}: "
                f"{C4_DECODE_STEPS if diverge is None else diverge} of {C4_DECODE_STEPS} tokens identical"
                + ("" if diverge is None else f", then a near-tie (oracle top-2 margin {margins[diverge]:.2e} * rms)")
                + f"; smallest oracle top-2 margin {min(margins):.2e} * rms; teacher-forced argmax differs at "
                f"{len(mism)} steps {mism} (reference -Ofast build: {len(ref_flips)} {ref_flips}); logits worst "
                f"{max(errs):.2e} * rms against tol {tol_rel:.2e} (reference builds' drift {drift:.2e}): ratio "
                f"{worst:.3f}; prompt K/V worst mean-flip/limit {kv_w:.3f} (reference builds' worst mean "
                f"{kv_ref:.4f}) ({time.perf_counter() - t0:.1f} s)")
            assert worst <= 1.0, f"logits: worst max|dlogit|/rms {max(errs):.3g} > {tol_rel:.3g}"
            if diverge is not None:
                assert margins[diverge] <= 2 * tol_rel, \
                    f"free-running greedy: step {diverge} token {free_gpu[diverge]} != oracle's {free_orc[diverge]} " \
                    f"with oracle top-2 margin {margins[diverge]:.3g} * rms > {2 * tol_rel:.3g}"
            assert near <= 1.0, f"teacher-forced argmax differs at a step that is no near-tie ({mism})"
            assert len(mism) <= 2 * len(ref_flips) + 2, \
                f"teacher-forced argmax differs at {len(mism)} steps {mism}, the reference build's at " \
                f"{len(ref_flips)} {ref_flips}"
            dec_lims = kv_bounds(ref["kv_end"], orc_end, nkv, S, 1024, 1024 + C4_DECODE_STEPS)
            dec_w, _ = check_kv(gpu_end, orc_end, dec_lims, nkv, S, 1024, 1024 + C4_DECODE_STEPS, "decode rows")
            log(f"llama3-8b: decode rows K/V worst mean-flip/limit {dec_w:.3f}")
        finally:
            m.close()


@pytest.fixture(scope="module")
def gemma2(torch_gpu, cpuref):
    """The Gemma-2-2B workload's model and prompt, and the reference's own
    drift on it under the gemma3 semantics its builds run: the oracle's
    prompt and 128 sampled steps (each fed the oracle's sampled token), the
    reference -Ofast build's logits and caches on the same steps."""
    t0 = time.perf_counter()
    with l3p.Context(0) as c0:
        img = synth.synthetic_model(qtype=synth.Q8_0, make_mat=synth.gpu_q8_0_maker(c0, torch_gpu, 77),
                                    **bench.GEMMA2_2B)
    m = cpuref.open_model(img)
    try:
        prompt = np.random.default_rng(6).integers(0, m.vocab, 512).astype(np.int32)
        m.prefill(prompt, 0, 511)
        orc_kv = all_kv(m.kv, m.n_layers)
        tok, pos, rng = int(prompt[-1]), 511, 42
        steps, rngs, lo_rs, toks = [], [], [], []
        for _ in range(C5_DECODE_STEPS):
            steps.append((tok, pos))
            rngs.append(rng)
            lo_r = m.forward(tok, pos)
            lo_rs.append(lo_r)
            tok, rng = cpuref.sample(lo_r, 0.9, 40, 0.9, rng)
            toks.append(tok)
            pos += 1
        info = {"n_layers": m.n_layers, "layer_bytes": int(orc_kv.shape[2]), "vocab": m.vocab}
        log(f"gemma2-2b: model {img.nbytes / 1e9:.2f} GB, oracle prompt and {len(steps)} sampled steps, reference "
            f"build running ({time.perf_counter() - t0:.1f} s)")
        ref = run_reference(img, info, prompt, 511, steps=steps)
        drift = max(float(np.max(np.abs(ref["logits"][i] - lo))) / rms(lo) for i, lo in enumerate(lo_rs))
        ref_mism = [i for i in range(len(steps)) if cpuref.sample(ref["logits"][i], 0.9, 40, 0.9, rngs[i])[0] != toks[i]]
        kv_lims = kv_bounds(ref["kv"], orc_kv, m.n_kv, m.seq_len, 0, 511)
        log(f"gemma2-2b: reference builds' drift {drift:.2e} * rms, sampled tokens differ at {len(ref_mism)} steps "
            f"({time.perf_counter() - t0:.1f} s)")
        yield dict(img=img, prompt=prompt, steps=steps, rngs=rngs, lo_rs=lo_rs, toks=toks, orc_kv=orc_kv,
                   tol_rel=max(1e-2, 2.0 * drift), drift=drift, ref_mism=ref_mism, kv_lims=kv_lims,
                   kv_ref=max(r[wv][2] for r in kv_lims for wv in (0, 1)))
    finally:
        m.close()


def sampled_steps(ctx, cpuref, steps, rngs, lo_rs, toks):
    """The GPU decodes the oracle's sampled steps; the device sampler is checked
    exactly on the GPU's own logits.  Returns the per-step logits errors
    (max|dlogit|/rms) and the steps whose sampled token differs."""
    errs, mism = [], []
    for step, ((tok, pos), rng) in enumerate(zip(steps, rngs)):
        tok_g, rng_g = ctx.decode(tok, pos, temperature=0.9, top_k=40, top_p=0.9, rng=rng)
        lo_g = ctx.logits()
        # the device sampler is the reference's sampler on the GPU's own logits
        assert (tok_g, rng_g) == cpuref.sample(lo_g, 0.9, 40, 0.9, rng), f"step {step}: device sampler"
        assert rng_g == cpuref.sample(lo_rs[step], 0.9, 40, 0.9, rng)[1], f"step {step}: RNG state"
        errs.append(float(np.max(np.abs(lo_g - lo_rs[step]))) / rms(lo_rs[step]))
        if tok_g != toks[step]:
            mism.append(step)
    return errs, mism


def test_gemma2_2b_prompt_and_sampled_decode(torch_gpu, cpuref, gemma2):
    """The reference's gemma3 semantics, on which its own builds set the drift."""
    t0 = time.perf_counter()
    g = gemma2
    with l3p.Context(0) as ctx:
        mi = ctx.load_gguf(g["img"])
        L, nkv, S = mi.n_layers, mi.n_kv_heads, mi.seq_len
        ctx.prefill(g["prompt"][:-1], 0)
        gpu_kv = all_kv(ctx.copy_kv, L)
        kv_w, _ = check_kv(gpu_kv, g["orc_kv"], g["kv_lims"], nkv, S, 0, 511, "prompt")
        errs, mism = sampled_steps(ctx, cpuref, g["steps"], g["rngs"], g["lo_rs"], g["toks"])
    worst = max(errs) / g["tol_rel"]
    log(f"gemma2-2b (gemma3 semantics): {C5_DECODE_STEPS} sampled steps, RNG states identical, device sampler "
        f"exact; sampled tokens differ from the oracle's at {len(mism)} steps {mism} (the reference's -Ofast build "
        f"at {len(g['ref_mism'])}); logits worst {max(errs):.2e} * rms against tol {g['tol_rel']:.2e} (reference "
        f"builds' drift {g['drift']:.2e}): ratio {worst:.3f}; prompt K/V worst mean-flip/limit {kv_w:.3f} "
        f"(reference builds' worst mean {g['kv_ref']:.4f}) ({time.perf_counter() - t0:.1f} s)")
    assert worst <= 1.0, f"logits: worst max|dlogit|/rms {max(errs):.3g} > {g['tol_rel']:.3g}"
    assert len(mism) <= 2 * len(g["ref_mism"]) + 2, \
        f"sampled tokens differ from the oracle's at {len(mism)} steps {mism}, the reference build's at " \
        f"{len(g['ref_mism'])} {g['ref_mism']}"


def test_gemma2_2b_as_benched(torch_gpu, cpuref, gemma2):
    """The workload exactly as bench.py runs it: alternating local/global
    layers and attention soft-cap 50 on both sides (load options
    swa_pattern=2, attn_softcap=50; the oracle's set_attention(2, 50)), the
    511-position prompt and 128 sampled steps, held to the tolerances the
    reference's builds set on the gemma3-semantics protocol of the same model
    (logits, K/V flip limits, twice the reference's sampled-token flips plus
    two)."""
    t0 = time.perf_counter()
    g = gemma2
    assert bench.GEMMA2_2B_LOAD == dict(swa_pattern=2, attn_softcap=50.0)
    m = cpuref.open_model(g["img"])
    try:
        m.set_attention(2, 50.0)
        prompt = g["prompt"]
        m.prefill(prompt, 0, 511)
        orc_kv = all_kv(m.kv, m.n_layers)
        tok, pos, rng = int(prompt[-1]), 511, 42
        steps, rngs, lo_rs, toks = [], [], [], []
        for _ in range(C5_DECODE_STEPS):
            steps.append((tok, pos))
            rngs.append(rng)
            lo_r = m.forward(tok, pos)
            lo_rs.append(lo_r)
            tok, rng = cpuref.sample(lo_r, 0.9, 40, 0.9, rng)
            toks.append(tok)
            pos += 1
    finally:
        m.close()
    # the options change the computation: the oracle's logits are not the gemma3 ones
    opt_shift = max(float(np.max(np.abs(a - b))) / rms(b) for a, b in zip(lo_rs[:4], g["lo_rs"][:4]))
    assert opt_shift > 0.0
    with l3p.Context(0) as ctx:
        mi = ctx.load_gguf(g["img"], **bench.GEMMA2_2B_LOAD)
        assert (mi.swa_pattern, mi.attn_softcap) == (2, 50.0)
        L, nkv, S = mi.n_layers, mi.n_kv_heads, mi.seq_len
        ctx.prefill(prompt[:-1], 0)
        gpu_kv = all_kv(ctx.copy_kv, L)
        kv_w, _ = check_kv(gpu_kv, orc_kv, g["kv_lims"], nkv, S, 0, 511, "prompt")
        errs, mism = sampled_steps(ctx, cpuref, steps, rngs, lo_rs, toks)
    worst = max(errs) / g["tol_rel"]
    log(f"gemma2-2b as benched (swa_pattern 2, attn_softcap 50): {C5_DECODE_STEPS} sampled steps, RNG states "
        f"identical, device sampler exact; sampled tokens differ from the oracle's at {len(mism)} steps {mism} "
        f"(limit {2 * len(g['ref_mism']) + 2}); logits worst {max(errs):.2e} * rms against tol {g['tol_rel']:.2e}: "
        f"ratio {worst:.3f}; prompt K/V worst mean-flip/limit {kv_w:.3f}; the options move the oracle's first logits "
        f"by {opt_shift:.2e} * rms ({time.perf_counter() - t0:.1f} s)")
    assert worst <= 1.0, f"logits: worst max|dlogit|/rms {max(errs):.3g} > {g['tol_rel']:.3g}"
    assert len(mism) <= 2 * len(g["ref_mism"]) + 2, \
        f"sampled tokens differ from the oracle's at {len(mism)} steps {mism}, the reference build's at " \
        f"{len(g['ref_mism'])} {g['ref_mism']}"
