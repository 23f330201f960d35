"""l3p_generate_greedy: the reference's greedy decode loop (c:5289-5309) with
the steps queued on the device ahead of the host's token reads.  Its tokens
must equal l3p_decode called step by step, which the model tests compare with
the oracle; stop ids end the run after the stop token, and a run continued
after a stop equals the uninterrupted one."""
import numpy as np
import pytest

import llama3pure_amd as l3p
from llama3pure_amd import synth

pytestmark = pytest.mark.gpu


def step_by_step(c, tok, pos, n):
    out = []
    for _ in range(n):
        tok, _ = c.decode(tok, pos, temperature=0.0)
        out.append(tok)
        pos += 1
    return out


@pytest.fixture(scope="module", params=["llama", "gemma3"])
def model_ctx(request, torch_gpu):
    """A fresh context per architecture: the first generate run captures its
    decode graphs inside the queued loop."""
    arch = request.param
    g = synth.synthetic_model(arch=arch, dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=512,
                              seed=21, tied=arch == "gemma3", softcap=30.0 if arch == "gemma3" else 0.0)
    c = l3p.Context(0)
    c.load_gguf(g)
    prompt = np.random.default_rng(3).integers(0, 512, 16).astype(np.int32)
    c.prefill(prompt[:-1], 0)
    yield arch, c, int(prompt[-1]), len(prompt) - 1
    c.close()


def test_generate_equals_step_by_step(model_ctx):
    arch, c, tok, pos = model_ctx
    # first through the queued loop (graphs captured there), then step by step
    # from the same state: steps at pos.. rewrite the cache rows they read
    gen = c.generate_greedy(tok, pos, 40)
    ref = step_by_step(c, tok, pos, 40)
    print(f"[generate] {arch}: {len(gen)} tokens, first {gen[:6]}", flush=True)
    assert gen == ref


def test_generate_across_attention_switch(model_ctx):
    """Positions 430..470 cross the switch from the per-head decode attention
    to chunks + merge (448 positions at head_dim < 192): two graph variants in
    one queued run."""
    arch, c, tok, _ = model_ctx
    gen = c.generate_greedy(tok, 430, 40)
    ref = step_by_step(c, tok, 430, 40)
    assert gen == ref


def test_generate_stop_and_continue(model_ctx):
    arch, c, tok, pos = model_ctx
    full = step_by_step(c, tok, pos, 30)
    j = 7
    stop = full[j]
    first = full.index(stop)   # the run ends at the first occurrence
    part = c.generate_greedy(tok, pos, 30, stop_ids=[stop, 100000])
    assert part == full[:first + 1]
    # continue after the stop: the step queued behind the stop token rewrote
    # the next position's cache rows with the same token
    rest = c.generate_greedy(part[-1], pos + len(part), 30 - len(part))
    assert part + rest == full


def test_generate_bounds(model_ctx):
    arch, c, tok, _ = model_ctx
    seq = c.model_info().seq_len
    assert len(c.generate_greedy(tok, seq - 3, 10)) == 3   # never past the context
    assert c.generate_greedy(tok, 5, 0) == []
    for bad in [dict(token=-1, pos=5, max_steps=4), dict(token=tok, pos=seq, max_steps=4),
                dict(token=tok, pos=5, max_steps=-1)]:
        with pytest.raises(l3p.L3PError) as e:
            c.generate_greedy(bad["token"], bad["pos"], bad["max_steps"])
        assert e.value.code == l3p.E_INVALID
