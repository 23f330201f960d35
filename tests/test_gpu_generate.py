"""l3p_generate_greedy and l3p_generate_sampled: the reference's decode loop
(c:5289-5309) with the steps queued on the device ahead of the host.  Greedy
steps read the previous argmax from device memory; sampled steps wait on the
device for the token the host's sampler finish hands over through pinned
memory.  Their tokens (and, sampled, the final RNG state) must equal
l3p_decode called step by step, which the model tests compare with the
oracle; stop ids end the run after the stop token, and a run continued after
a stop equals the uninterrupted one."""
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


def sampled_step_by_step(c, tok, pos, n, rng, **smp):
    out = []
    for _ in range(n):
        tok, rng = c.decode(tok, pos, rng=rng, **smp)
        out.append(tok)
        pos += 1
    return out, rng


SAMPLERS = [dict(temperature=0.9, top_k=40, top_p=0.9), dict(temperature=1.3, top_k=200, top_p=1.0),
            dict(temperature=0.5, top_k=1, top_p=0.5)]


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


@pytest.mark.parametrize("smp", SAMPLERS, ids=["t0.9_k40_p0.9", "t1.3_k200_p1", "t0.5_k1"])
def test_sampled_equals_step_by_step(model_ctx, smp):
    """Queued sampled steps give l3p_decode's tokens and final RNG state; the
    second half of the run crosses the attention-path switch at 448
    positions, and a second call (later sequence numbers) repeats the first."""
    arch, c, tok, pos = model_ctx
    for p0 in (pos, 420):
        gen, rng_g = c.generate_sampled(tok, p0, 48, rng=0x9E3779B97F4A7C15, **smp)
        ref, rng_r = sampled_step_by_step(c, tok, p0, 48, 0x9E3779B97F4A7C15, **smp)
        assert (gen, rng_g) == (ref, rng_r), (arch, p0, smp)
        again, rng_a = c.generate_sampled(tok, p0, 48, rng=0x9E3779B97F4A7C15, **smp)
        assert (again, rng_a) == (gen, rng_g)
    print(f"[generate] {arch} sampled {smp}: first {gen[:6]}", flush=True)


def test_sampled_stop_and_continue(model_ctx):
    arch, c, tok, pos = model_ctx
    smp = SAMPLERS[0]
    full, rng_full = sampled_step_by_step(c, tok, pos, 30, 12345, **smp)
    stop = full[9]
    first = full.index(stop)
    part, rng_p = c.generate_sampled(tok, pos, 30, rng=12345, stop_ids=[100000, stop], **smp)
    assert part == full[:first + 1]
    rest, rng_r = c.generate_sampled(part[-1], pos + len(part), 30 - len(part), rng=rng_p, **smp)
    assert part + rest == full and rng_r == rng_full


def test_sampled_bounds(model_ctx):
    arch, c, tok, _ = model_ctx
    seq = c.model_info().seq_len
    assert len(c.generate_sampled(tok, seq - 3, 10, rng=7)[0]) == 3   # never past the context
    assert c.generate_sampled(tok, 5, 0, rng=7) == ([], 7)
    for bad in [dict(token=-1, pos=5, max_steps=4), dict(token=tok, pos=seq, max_steps=4),
                dict(token=tok, pos=5, max_steps=-1), dict(token=tok, pos=5, max_steps=4, temperature=0.0),
                dict(token=tok, pos=5, max_steps=4, top_k=0)]:
        kw = dict(bad)
        with pytest.raises(l3p.L3PError) as e:
            c.generate_sampled(kw.pop("token"), kw.pop("pos"), kw.pop("max_steps"), rng=7, **kw)
        assert e.value.code == l3p.E_INVALID, bad
    # the context still works after the refused calls; top_k above the
    # vocabulary keeps every logit (c:4815-4816)
    smp = dict(temperature=0.9, top_k=600, top_p=0.95)
    assert c.generate_sampled(tok, 5, 4, rng=7, **smp) == sampled_step_by_step(c, tok, 5, 4, 7, **smp)
