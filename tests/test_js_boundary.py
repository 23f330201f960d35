"""The JS boundary: the N-API addon and js/llama3pure_amd.js driven by Node
the way the reference's generate() drives its engine."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from llama3pure_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "js", "l3p_napi.node")
NODE = shutil.which("node") or shutil.which("nodejs")

needs_node = pytest.mark.skipif(not NODE or not os.path.exists(ADDON), reason="node or the built addon is missing")


@needs_node
def test_addon_exports_and_error_mapping():
    """Loads without a GPU; a failing call throws an Error carrying l3p's message and code."""
    code = ("var m = require(process.argv[1]);"
            "var names = Object.keys(m.addon).sort();"
            "var r = {names: names};"
            "try { m.addon.loadGguf(null, new Uint8Array(4), 0) } catch (e) { r.bad = e.message }"
            "console.log(JSON.stringify(r))")
    r = subprocess.run([NODE, "-e", code, os.path.join(ROOT, "js", "llama3pure_amd.js")], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["names"] == sorted(["open", "close", "loadGguf", "transformer", "transformerPrefill", "decode",
                                   "sample", "setSeed", "getSeed"])
    assert "engine handle" in res["bad"]


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("arch", ["llama", "gemma3"])
def test_js_generate_flow_matches_oracle(arch, tmp_path, cpuref):
    """Prefill + greedy steps through the JS boundary: the logits match the
    oracle within the single-model tolerance and the tokens are the oracle's."""
    extra = dict(head_dim=256, softcap=30.0, swa_window=16, tied=True) if arch == "gemma3" else {}
    g = synth.synthetic_model(arch=arch, dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv=2, vocab=2048, ctx=128,
                              qtype=synth.Q8_0, seed=31, norm_jitter=0.1, **extra)
    p = tmp_path / "m.gguf"
    p.write_bytes(g)
    prompt = np.random.default_rng(4).integers(0, 2048, 40).astype(np.int32)
    steps = 8
    out = tmp_path / "out.bin"
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "js_run.js"), str(p), str(out),
                        ",".join(map(str, prompt)), str(steps)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    raw = np.fromfile(out, np.uint8).reshape(steps, 2048 * 4 + 4)
    m = cpuref.open_model(g)
    pos = 0
    while pos < len(prompt) - 1:
        bs = min(32, len(prompt) - 1 - pos)
        m.prefill(prompt, pos, bs)
        pos += bs
    tok = int(prompt[-1])
    for s in range(steps):
        lo = m.forward(tok, pos)
        lj = raw[s, :2048 * 4].view(np.float32)
        rms = float(np.sqrt(np.mean(lo.astype(np.float64) ** 2)))
        assert float(np.abs(lj - lo).max()) <= 1e-2 * rms, (arch, s)
        tj = int(raw[s, 2048 * 4:].view(np.int32)[0])
        assert tj == int(np.argmax(lj))
        tok, pos = tj, pos + 1
    m.close()
