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
@pytest.mark.parametrize("arch", ["llama", "gemma3", "gemma3_opts"])
def test_js_generate_flow_matches_oracle(arch, tmp_path, cpuref):
    """Prefill + greedy steps through the JS boundary: the logits match the
    oracle within the single-model tolerance and the tokens are the oracle's.
    gemma3_opts passes the load options swaPattern 2 and attnSoftcap 5 (a cap
    low enough to change the scores) through Engine.load, and the oracle runs
    with the same options."""
    extra = dict(head_dim=256, softcap=30.0, swa_window=16, tied=True) if arch.startswith("gemma3") else {}
    g = synth.synthetic_model(arch=arch.split("_")[0], dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv=2,
                              vocab=2048, ctx=128, qtype=synth.Q8_0, seed=31, norm_jitter=0.1, **extra)
    p = tmp_path / "m.gguf"
    p.write_bytes(g)
    prompt = np.random.default_rng(4).integers(0, 2048, 40).astype(np.int32)
    steps = 8
    out = tmp_path / "out.bin"
    opts = ["2", "5.0"] if arch == "gemma3_opts" else []
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "js_run.js"), str(p), str(out),
                        ",".join(map(str, prompt)), str(steps)] + opts, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    info = json.loads(r.stdout.strip().splitlines()[-1])
    if opts:
        assert info["swaPattern"] == 2 and abs(info["attnSoftcap"] - 5.0) < 1e-6, info
    raw = np.fromfile(out, np.uint8).reshape(steps, 2048 * 4 + 4)
    m = cpuref.open_model(g)
    if opts:
        m.set_attention(2, 5.0)
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


# --------------------------------------------------------------------------
# js/llama3pure.js: the reference's llama3pure({type}) entry point
# (llama3pure-js-engine.js:7033-7260) over the device engine.

SHIM_RUN = os.path.join(ROOT, "tests", "js_shim_run.js")
CYCLE = [100 + i for i in range(10)]


def cycle_model():
    """A one-layer Llama-layout model whose greedy successor of token 100 + i
    is 100 + (i + 1) % 10: every block matrix is zero, so the residual is the
    token's embedding, which for the ten cycle tokens is the unit vector e_i;
    the output row of 100 + (i + 1) % 10 is e_i and every other output row is
    zero, so after the final RMSNorm (x / rms = 16 e_i at dim 256) the
    successor's logit is ~16 and every other logit is 0."""
    dim, hidden, vocab = 256, 512, 512
    emb = np.random.default_rng(0).normal(0, 0.02, (vocab, dim)).astype(np.float32)
    out = np.zeros((vocab, dim), np.float32)
    for i in range(10):
        emb[CYCLE[i]] = 0.0
        emb[CYCLE[i], i] = 1.0
        out[CYCLE[(i + 1) % 10], i] = 1.0
    hd = dim // 8
    zeros = {"attn_q": (8 * hd, dim), "attn_k": (2 * hd, dim), "attn_v": (2 * hd, dim),
             "attn_output": (dim, 8 * hd), "ffn_gate": (hidden, dim), "ffn_up": (hidden, dim),
             "ffn_down": (dim, hidden)}
    mats = {f"blk.0.{k}.weight": np.zeros(s, np.float32) for k, s in zeros.items()}
    mats["token_embd.weight"] = emb
    mats["output.weight"] = out
    return synth.synthetic_model(arch="llama", dim=dim, hidden=hidden, n_layers=1, n_heads=8, n_kv=2, vocab=vocab,
                                 ctx=256, qtype=synth.Q8_0, seed=5, mats=mats)


def run_shim(tmp_path, model, scenarios):
    p = tmp_path / "m.gguf"
    p.write_bytes(model)
    s = tmp_path / "sc.json"
    s.write_text(json.dumps(scenarios))
    r = subprocess.run([NODE, SHIM_RUN, str(p), str(s)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def check_messages(res):
    """'loaded', then one 'token' message per cbRender piece in the same
    order, then 'complete' with their concatenation."""
    msgs, render = res["msgs"], res["render"]
    assert msgs[0] == {"type": "loaded"}
    assert msgs[-1]["type"] == "complete"
    toks = msgs[1:-1]
    assert all(m["type"] == "token" for m in toks)
    assert [m["token"] for m in toks] == render
    assert msgs[-1]["output"] == "".join(render)


def pieces(ids):
    return [f"<{i}>" for i in ids]


@needs_node
@pytest.mark.gpu
def test_js_shim_stop_rules_and_messages(tmp_path):
    """eos/eot stops, the absolute maxTokens cap, newline holding and the
    10-gram repetition stop (js:7066-7158) on the cycle model, whose greedy
    continuation of a prompt ending in 100 is 101, 102, ..., 109, 100, ..."""
    prompt = [5, 6, 7, 8, 100]   # generation starts at position 4
    sc = [
        dict(prompt=prompt, maxTokens=12),            # positions 4..11: eight tokens
        dict(prompt=prompt, eos=105),                 # stops before 105
        dict(prompt=prompt, eot=103),                 # stops before 103
        dict(prompt=prompt, newline=102, eos=104),    # "\n" emitted before the next piece
        dict(prompt=prompt, newline=103, eos=104),    # a held "\n" before the end is dropped
        dict(prompt=prompt),                          # repetition stop
        dict(prompt=prompt, maxTokens=3),             # cap below the prompt: nothing generated
        dict(prompt=prompt, maxTokens=-5, eos=102),   # maxTokens <= 0: the context length
    ]
    res = run_shim(tmp_path, cycle_model(), sc)
    for r in res:
        assert r["errors"] == [], r["errors"]
        check_messages(r)
    assert res[0]["render"] == pieces(range(101, 109))
    assert res[1]["render"] == pieces(range(101, 105))
    assert res[2]["render"] == pieces([101, 102])
    assert res[3]["render"] == ["<101>", "\n", "<103>"]
    assert res[4]["render"] == ["<101>", "<102>"]
    # 10-token cycle: at position p (p % 10 == 0) with L = p - 3 tokens
    # generated, the last 10 match the 6 windows before them once L >= 70,
    # i.e. first at p = 80, after 77 tokens
    assert res[5]["render"] == pieces([CYCLE[(k + 1) % 10] for k in range(77)])
    assert res[6]["render"] == []
    assert res[7]["render"] == ["<101>"]


@needs_node
@pytest.mark.gpu
def test_js_shim_load_error_is_logged(tmp_path):
    """A bad GGUF in the load message is caught and logged (js:7246-7248):
    no 'loaded' message, and generate does nothing."""
    res = run_shim(tmp_path, cycle_model(), [dict(prompt=[1, 100], badModel=True)])[0]
    assert res["msgs"] == [] and res["render"] == []
    assert len(res["errors"]) == 1, res["errors"]
    assert "Unsupported GGUF version: 9" in res["errors"][0] and "(code -5)" in res["errors"][0], res["errors"]


@needs_node
@pytest.mark.gpu
def test_js_shim_greedy_matches_oracle(tmp_path, cpuref):
    """The shim's coalesced prefill and device decode steps give the oracle's
    greedy tokens (until a near-tie the reference's own builds may resolve
    either way)."""
    g = synth.synthetic_model(arch="llama", dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv=2, vocab=2048, ctx=128,
                              qtype=synth.Q8_0, seed=31, norm_jitter=0.1)
    prompt = [int(t) for t in np.random.default_rng(4).integers(3, 2048, 40)]
    steps = 12
    res = run_shim(tmp_path, g, [dict(prompt=prompt, maxTokens=len(prompt) - 1 + steps)])[0]
    assert res["errors"] == []
    check_messages(res)
    got = [int(p[1:-1]) for p in res["render"]]
    assert len(got) == steps
    m = cpuref.open_model(g)
    m.prefill(np.array(prompt, np.int32), 0, len(prompt) - 1)
    tok, pos, same = prompt[-1], len(prompt) - 1, 0
    for s in range(steps):
        lo = m.forward(tok, pos)
        want = int(np.argmax(lo))
        if got[s] != want:
            top = np.sort(lo)
            rms = float(np.sqrt(np.mean(lo.astype(np.float64) ** 2)))
            assert float(top[-1] - top[-2]) <= 2e-2 * rms, (s, got[s], want)
            break
        same += 1
        tok, pos = want, pos + 1
    m.close()
    print(f"[js shim] {same} of {steps} greedy steps identical; load + generate {res['ms']} ms", flush=True)
