"""Writes ref_drift.json: how far the reference engine's own optimised build
(Makefile "fast"/OpenMP line: gcc -Ofast -fopenmp, which vectorises and
reorders its fp32 sums) drifts from its plain build (bit-identical to the
oracle) on the synthetic models of test_gpu_model.py: the full models under
the teacher-forced protocol of test_teacher_forced_logits_and_kv, and the
one-layer models of test_single_layer_position0_tight per token.

The GPU path reorders fp32 sums too, so its logits are held to a tolerance
derived from this drift: it may differ from the oracle by as much as the
reference differs from itself across its own supported builds.

Needs oracle/_ref/libref_omp.so (``make -C oracle ref``).  One model per
subprocess because the reference keeps its model in process globals.

usage: python tests/golden/make_ref_drift.py              (rewrites ref_drift.json)
       python tests/golden/make_ref_drift.py --long-only  (refreshes its "long" section)
"""
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

STEPS = 24


def measure(name: str) -> dict:
    import oracle
    from llama3pure_amd import synth
    import model_cases as T

    g = synth.synthetic_model(**T.MODELS[name])
    fd, path = tempfile.mkstemp(suffix=".gguf")
    with os.fdopen(fd, "wb") as f:
        f.write(g)
    try:
        ref = oracle.Ref(oracle.REF_OMP_SO)
        assert ref.lib.ref_model_open(path.encode(), 0) == 0
        m = oracle.CpuRef().open_model(g)
        prompt = T.teacher_prompt(m)
        n = len(prompt) - 1
        pos = 0
        while pos < n:  # the reference's prefill batches of 32 (c:5277-5287)
            bs = min(32, n - pos)
            ref.lib.ref_prefill(oracle._vp(prompt), pos, bs)
            m.prefill(prompt, pos, bs)
            pos += bs
        tok = int(prompt[-1])
        out = np.empty(m.vocab, np.float32)
        rel = []
        for _ in range(STEPS):
            lo = m.forward(tok, pos)
            ref.lib.ref_forward(tok, pos, 1, oracle._vp(out))
            rel.append(float(np.abs(lo - out).max()) / T.rms(lo))
            tok, pos = int(np.argmax(lo)), pos + 1
        kv = {}
        for layer in (0, m.n_layers - 1):
            for wv in (0, 1):
                b = m.kv(layer, bool(wv))
                a = np.empty(b.size, np.uint8)
                ref.lib.ref_copy_kv(layer, wv, oracle._vp(a), a.size)
                d = T.kv_quant_diff(a, b, m, pos)
                kv[f"{layer}/{'v' if wv else 'k'}"] = {"max": int(d.max()), "mean": float(d.mean())}
        return {"max_rel": max(rel), "per_step": rel, "kv": kv}
    finally:
        os.unlink(path)


def measure_single(case: str) -> list:
    """Per token of SINGLE_TOKENS: max|dlogit|/rms of the reference's two
    builds on the one-layer model `case` at position 0."""
    import oracle
    import model_cases as T

    g = T.single_layer_model(case)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    with os.fdopen(fd, "wb") as f:
        f.write(g)
    try:
        ref = oracle.Ref(oracle.REF_OMP_SO)
        assert ref.lib.ref_model_open(path.encode(), 0) == 0
        m = oracle.CpuRef().open_model(g)
        out = np.empty(m.vocab, np.float32)
        rel = []
        for tok in T.SINGLE_TOKENS:
            lo = m.forward(tok, 0)
            ref.lib.ref_forward(tok, 0, 1, oracle._vp(out))
            rel.append(float(np.abs(lo - out).max()) / T.rms(lo))
        return rel
    finally:
        os.unlink(path)


def measure_long(case: str) -> dict:
    """The long-context protocol of test_gpu_long_context.py: a prompt of
    LONG_CASES[case]["prompt"] tokens (the reference's prefill batches of 32,
    c:5277-5287), then LONG_STEPS teacher-forced decode steps; per step
    max|dlogit|/rms of the reference's two builds, and the K/V quant
    differences of every layer over all positions written."""
    import oracle
    from llama3pure_amd import synth
    import model_cases as T

    c = T.LONG_CASES[case]
    g = synth.synthetic_model(**c["model"])
    fd, path = tempfile.mkstemp(suffix=".gguf")
    with os.fdopen(fd, "wb") as f:
        f.write(g)
    try:
        ref = oracle.Ref(oracle.REF_OMP_SO)
        assert ref.lib.ref_model_open(path.encode(), 0) == 0
        m = oracle.CpuRef().open_model(g)
        toks = T.long_prompt(case)
        n = c["prompt"]
        pos = 0
        while pos < n:
            bs = min(32, n - pos)
            ref.lib.ref_prefill(oracle._vp(toks), pos, bs)
            pos += bs
        m.prefill(toks, 0, n)
        tok = int(toks[n])
        out = np.empty(m.vocab, np.float32)
        rel = []
        for _ in range(T.LONG_STEPS):
            lo = m.forward(tok, pos)
            ref.lib.ref_forward(tok, pos, 1, oracle._vp(out))
            rel.append(float(np.abs(lo - out).max()) / T.rms(lo))
            tok, pos = int(np.argmax(lo)), pos + 1
        kv = {}
        for layer in range(m.n_layers):
            for wv in (0, 1):
                b = m.kv(layer, bool(wv))
                a = np.empty(b.size, np.uint8)
                ref.lib.ref_copy_kv(layer, wv, oracle._vp(a), a.size)
                d = T.kv_quant_diff(a, b, m, pos)
                kv[f"{layer}/{'v' if wv else 'k'}"] = {"max": int(d.max()), "mean": float(d.mean())}
        return {"max_rel": max(rel), "per_step": rel, "kv": kv}
    finally:
        os.unlink(path)


def main():
    if len(sys.argv) == 3 and sys.argv[1] == "--long":
        print(json.dumps(measure_long(sys.argv[2])))
        return
    if len(sys.argv) == 2 and sys.argv[1] == "--long-only":
        # refresh only the long-context section of an existing ref_drift.json
        import model_cases as T
        path = os.path.join(HERE, "ref_drift.json")
        with open(path) as f:
            out = json.load(f)
        out["long"] = long_section(T)
        with open(path, "w") as f:
            json.dump(out, f, indent=1)
        return
    if len(sys.argv) == 3 and sys.argv[1] == "--one":
        print(json.dumps(measure(sys.argv[2])))
        return
    if len(sys.argv) == 3 and sys.argv[1] == "--single":
        print(json.dumps(measure_single(sys.argv[2])))
        return
    import model_cases as T

    out = {"build": "gcc -Ofast -fopenmp -march=x86-64-v3 (reference Makefile OpenMP line)",
           "protocol": f"teacher-forced, prompt of 20, {STEPS} decode steps; max|dlogit|/rms(logits)",
           "models": {}}
    env = dict(os.environ, OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "4"))
    for name in T.MODELS:
        r = subprocess.run([sys.executable, __file__, "--one", name], check=True, capture_output=True, text=True,
                           env=env)
        out["models"][name] = json.loads(r.stdout.strip().splitlines()[-1])
        print(name, f"{out['models'][name]['max_rel']:.3e}")
    out["single_layer"] = {}
    for case in T.SINGLE_LAYER:
        r = subprocess.run([sys.executable, __file__, "--single", case], check=True, capture_output=True, text=True,
                           env=env)
        out["single_layer"][case] = json.loads(r.stdout.strip().splitlines()[-1])
        print(case, " ".join(f"{v:.1e}" for v in out["single_layer"][case]))
    out["long"] = long_section(T)
    with open(os.path.join(HERE, "ref_drift.json"), "w") as f:
        json.dump(out, f, indent=1)


def long_section(T) -> dict:
    env = dict(os.environ, OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "4"))
    res = {}
    for case in T.LONG_CASES:
        r = subprocess.run([sys.executable, __file__, "--long", case], check=True, capture_output=True, text=True,
                           env=env)
        res[case] = json.loads(r.stdout.strip().splitlines()[-1])
        print(case, f"{res[case]['max_rel']:.3e}",
              "kv max", max(v["max"] for v in res[case]["kv"].values()),
              "mean", f"{max(v['mean'] for v in res[case]['kv'].values()):.2e}")
    return res


if __name__ == "__main__":
    main()
