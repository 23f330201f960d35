"""GPU decode/prefill parity against the oracle on seeded synthetic models.

The oracle's forward is bit-identical to the reference engine's
(tests/test_oracle_model.py), so these compare the HIP path with the
reference's arithmetic.  GEMVs sum in a different fp32 order, so values
differ in their last bits; where such a value is quantized (the Q8_0 K/V/Q
blocks, the truncated fp16 block scales, the Q8_0 activations of Q4_0
weights) a last-bit difference occasionally moves a quant by one step or a
scale by one fp16 ulp (2^-10 relative).  The stated tolerances:

  * single layer at position 0 (no attention history), per token:
        |logit_gpu - logit_oracle| <= max(1e-4, 2 * drift) * rms(logits)
    with drift the reference's own build-to-build difference on that token
    (~5e-7 unless a quantized value sits on a rounding boundary);
  * full models after prefill:
        |logit_gpu - logit_oracle| <= max(1e-2, 2 * drift) * rms(logits)
    where drift is the largest max|dlogit|/rms by which the reference's own
    optimised build (gcc -Ofast -fopenmp, its Makefile's OpenMP line) departs
    from its plain build on the same model and protocol
    (tests/golden/ref_drift.json, written by tests/golden/make_ref_drift.py);
  * KV cache: every quant within 1 of the oracle's (or one more than the
    largest difference between the reference's two builds) and >= 99%
    identical (or a mean difference within three times that between the
    reference's builds: in Q4_0 models every activation is re-quantized to
    Q8_0, so one early rounding event, which either side may take, moves
    many later quants; the reference's builds show the same spread);
  * greedy tokens identical for 32 free-running steps, or until a step whose
    oracle top-2 margin is within 2 * tolerance (a near-tie that the
    reference's own builds may also resolve either way), and in any case
    for at least the first GREEDY_MIN_SAME steps.

Norm weights are jittered around 1.0 as in trained models; with all-ones
norms and Q4_0 embeddings the activations fall exactly on Q8_0 rounding ties,
where last-bit differences flip many quants (the reference's own C and JS
engines differ there too).
"""
import numpy as np
import pytest

import llama3pure_amd as l3p
from llama3pure_amd import synth
from model_cases import (MODELS, REF_DRIFT, SINGLE_DRIFT, SINGLE_LAYER, SINGLE_TOKENS, kv_quant_diff, rms,
                         single_layer_model, teacher_prompt)

pytestmark = pytest.mark.gpu

# free-running greedy steps that must be identical before a near-tie may end
# the comparison (every case ran 32 of 32 when this was set)
GREEDY_MIN_SAME = 16


def tol_of(lo, name):
    return max(1e-2, 2.0 * REF_DRIFT[name]["max_rel"]) * rms(lo)


def margin(lo):
    s = np.sort(lo)
    return float(s[-1] - s[-2])


@pytest.fixture(scope="module", params=list(MODELS))
def pair(request, ctx, cpuref):
    kw = MODELS[request.param]
    g = synth.synthetic_model(**kw)
    ctx.load_gguf(g)
    m = cpuref.open_model(g)
    yield request.param, g, m
    m.close()


def test_model_info(pair, ctx):
    name, g, m = pair
    mi = ctx.model_info()
    assert (mi.dim, mi.n_layers, mi.n_heads, mi.n_kv_heads, mi.vocab_size, mi.seq_len, mi.head_dim) == \
        (m.dim, m.n_layers, m.n_heads, m.n_kv, m.vocab, m.seq_len, m.head_dim)
    assert mi.is_gemma == m.is_gemma


def test_rope_tables_bit_exact(pair, ctx):
    """The library's host-built RoPE rows equal the oracle's (c:381-422)."""
    name, g, m = pair
    for swa in ((False, True) if m.is_gemma else (False,)):
        for pos in (0, 1, 7, 100, m.seq_len - 1):
            c, s = ctx.rope_row(swa, pos)
            rc, rs = m.rope_row(swa, pos)
            assert np.array_equal(c.view(np.uint32), rc.view(np.uint32))
            assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("case", list(SINGLE_LAYER))
def test_single_layer_position0_tight(torch_gpu, cpuref, case):
    """No attention history and one layer: only fp32 summation order differs.

    Per token, max|dlogit| <= max(1e-4, 2 * drift) * rms(logits), where drift
    is what the reference's -Ofast -fopenmp build shows against its plain
    build on the same token (tests/golden/ref_drift.json, "single_layer").
    The drift is ~5e-7 except where a quantized value (a Q8_0 activation of
    Q4_0 weights, a K/V quant) sits on a rounding boundary; there either build
    may round one step the other way and logits move by up to a few percent."""
    g = single_layer_model(case)
    drift = SINGLE_DRIFT[case]
    with l3p.Context(0) as c2:
        c2.load_gguf(g)
        m = cpuref.open_model(g)
        rel = []
        for tok in SINGLE_TOKENS:
            a = m.forward(tok, 0)
            b = c2.forward(tok, 0)
            rel.append(float(np.max(np.abs(a - b))) / rms(a))
        m.close()
    for tok, r, d in zip(SINGLE_TOKENS, rel, drift):
        assert r <= max(1e-4, 2.0 * d), (case, tok, r, d)


def test_teacher_forced_logits_and_kv(pair, ctx):
    """Prefill then decode with the oracle's greedy tokens fed to both sides."""
    name, g, m = pair
    prompt = teacher_prompt(m)
    ctx.prefill(prompt[:-1], 0)
    m.prefill(prompt[:-1], 0, len(prompt) - 1)
    tok, pos = int(prompt[-1]), len(prompt) - 1
    worst = 0.0
    for step in range(24):
        lo_ref = m.forward(tok, pos)
        lo_gpu = ctx.forward(tok, pos)
        tol = tol_of(lo_ref, name)
        err = float(np.max(np.abs(lo_gpu - lo_ref)))
        worst = max(worst, err / tol)
        assert err <= tol, f"{name} step {step}: max |dlogit| {err:.3g} > {tol:.3g}"
        if margin(lo_ref) > 2 * tol:
            assert int(np.argmax(lo_gpu)) == int(np.argmax(lo_ref))
        tok, pos = int(np.argmax(lo_ref)), pos + 1
    # KV cache: the same Q8_0 blocks up to one-step flips, or as close as the
    # reference's two builds are to each other
    for layer in (0, m.n_layers - 1):
        for wv in (False, True):
            d = kv_quant_diff(ctx.copy_kv(layer, wv), m.kv(layer, wv), m, pos)
            r = REF_DRIFT[name]["kv"][f"{layer}/{'v' if wv else 'k'}"]
            lim = max(0.01, 3.0 * r["mean"])
            print(f"[teacher] {name} layer {layer} {'v' if wv else 'k'}: flip rate {float(d.mean()):.5f} "
                  f"(limit {lim:.5f}, reference builds {r['mean']:.5f}), max step {int(d.max())}; "
                  f"logits worst {worst:.3f} of tolerance", flush=True)
            assert d.max() <= max(1, r["max"] + 1) and d.mean() <= lim, \
                (name, layer, wv, int(d.max()), float(d.mean()), r)


def test_greedy_decode_identical(pair, ctx):
    """Free-running greedy decode: same tokens as the oracle for 32 steps,
    or up to a near-tie after at least GREEDY_MIN_SAME identical steps."""
    name, g, m = pair
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, m.vocab, 12).astype(np.int32)
    ctx.prefill(prompt[:-1], 0)
    m.prefill(prompt[:-1], 0, len(prompt) - 1)
    t_gpu = t_ref = int(prompt[-1])
    pos = len(prompt) - 1
    same = 0
    for step in range(32):
        t_gpu, _ = ctx.decode(t_gpu, pos, temperature=0.0)
        lo = m.forward(t_ref, pos)
        t_ref = int(np.argmax(lo))
        if t_gpu != t_ref:
            assert margin(lo) <= 2 * tol_of(lo, name), \
                f"{name} step {step}: token {t_gpu} != {t_ref} with top-2 margin {margin(lo):.3g}"
            assert step >= GREEDY_MIN_SAME, \
                f"{name}: tokens differ at step {step}, before {GREEDY_MIN_SAME} identical steps (a near-tie)"
            break
        same += 1
        pos += 1
    print(f"[greedy] {name}: {same} of 32 steps identical"
          + ("" if same == 32 else f", then a near tie (top-2 margin {margin(lo):.3g})"), flush=True)


def test_sampler_matches_oracle(pair, ctx, cpuref, torch_gpu):
    """Top-k/top-p sampling on identical logits picks the oracle's token."""
    name, g, m = pair
    rng = np.random.default_rng(13)
    seed = 0x9E3779B97F4A7C15
    for trial in range(20):
        lo = (rng.standard_normal(m.vocab) * 3).astype(np.float32)
        d = torch_gpu.from_numpy(lo).cuda()
        k = [1, 5, 40, 100][trial % 4]
        p = [0.9, 1.0, 0.5, 0.95][trial % 4]
        t_gpu, s_gpu = ctx.sample(d, m.vocab, temperature=0.9, top_k=k, top_p=p, rng=seed)
        t_ref, s_ref = cpuref.sample(lo, 0.9, k, p, seed)
        assert s_gpu == s_ref
        assert t_gpu == t_ref, (trial, k, p)
        seed = s_ref
    t_gpu, _ = ctx.sample(torch_gpu.from_numpy(lo).cuda(), m.vocab, temperature=0.0)
    assert t_gpu == int(np.argmax(lo))


@pytest.mark.parametrize("vocab", [128256, 256000])
def test_sampler_full_vocab(torch_gpu, cpuref, vocab):
    """Top-k/top-p over full-size vocabularies (several LDS blocks of the
    top-k scan) picks the oracle's token and RNG state: normal logits, logits
    rounded to halves (many ties, so the lowest-slot rule decides),
    increasing logits (every index replaces a slot), and NaN logits past
    the initial slots."""
    g = synth.synthetic_model(arch="llama", dim=64, hidden=64, n_layers=1, n_heads=2, n_kv=1, vocab=vocab, ctx=32,
                              qtype=synth.Q8_0, seed=vocab % 1000)
    rng = np.random.default_rng(vocab)
    seed = 0x9E3779B97F4A7C15
    with l3p.Context(0) as c:
        c.load_gguf(g)
        for trial in range(12):
            lo = (rng.standard_normal(vocab) * 3).astype(np.float32)
            if trial % 3 == 1:
                lo = (np.round(lo * 2) / 2).astype(np.float32)
            elif trial % 3 == 2:
                lo = np.sort(lo)
            if trial in (1, 7, 9):   # NaN logits past the initial slots: never inserted
                lo[rng.integers(1000, vocab, 50)] = np.nan
            k = [1, 40, 1000, 100, 200, 65][trial % 6]   # one to sixteen slot rows of 64
            p = [0.9, 1.0, 0.95, 0.5][trial % 4]
            t_gpu, s_gpu = c.sample(torch_gpu.from_numpy(lo).cuda(), vocab, temperature=0.9, top_k=k, top_p=p,
                                    rng=seed)
            t_ref, s_ref = cpuref.sample(lo, 0.9, k, p, seed)
            assert (t_gpu, s_gpu) == (t_ref, s_ref), (vocab, trial, k, p)
            seed = s_ref


def test_graph_replay_equals_eager(torch_gpu):
    """From the second step on, the layer stack replays a captured HIP graph.
    Every replay must give exactly the eager logits and KV cache; the eager
    reference is a context with launch timing on (which runs eagerly), and
    unrelated eager GEMVs run between the replays."""
    g = synth.synthetic_model(**dict(MODELS["gemma_q8_0"], n_layers=3))
    rng = np.random.default_rng(14)
    toks = rng.integers(0, 2048, 24).astype(np.int32)
    w = torch_gpu.from_numpy(synth.random_blocks(synth.Q8_0, 256, 512, seed=3)).cuda()
    xg = torch_gpu.from_numpy(synth.random_x(512, seed=4)).cuda()
    yg = torch_gpu.empty(256, device="cuda")
    with l3p.Context(0) as eager, l3p.Context(0) as graphed:
        eager.load_gguf(g)
        graphed.load_gguf(g)
        eager.profile(True)
        for c in (eager, graphed):
            c.prefill(toks[:16], 0)
        for i in range(16, 24):
            a = eager.forward(int(toks[i]), i)
            graphed.gemv(synth.Q8_0, w, 256, 512, xg, yg)       # eager work between replays
            b = graphed.forward(int(toks[i]), i)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}"
        for layer in range(3):
            for wv in (False, True):
                assert np.array_equal(eager.copy_kv(layer, wv), graphed.copy_kv(layer, wv))


@pytest.mark.parametrize("dim,heads,kv", [(256, 8, 8), (768, 8, 4), (512, 16, 1), (256, 4, 1)])
def test_head_shapes(torch_gpu, cpuref, dim, heads, kv):
    """Head sizes 32, 96, 32 and 64 with KV groups of 1, 2, 16 and 4 heads,
    across more than one 64-position chunk: logits within the full-model
    tolerance and the layer-0 KV cache equal up to one-step quant flips (the
    K/V projections sum in another fp32 order, so a value on a rounding
    boundary may quantize one step apart)."""
    g = synth.synthetic_model(arch="llama", dim=dim, hidden=256, n_layers=2, n_heads=heads, n_kv=kv, vocab=512,
                              ctx=256, qtype=synth.Q8_0, seed=dim + heads, norm_jitter=0.1)
    toks = np.random.default_rng(dim).integers(0, 512, 75).astype(np.int32)
    with l3p.Context(0) as c2:
        c2.load_gguf(g)
        m = cpuref.open_model(g)
        c2.prefill(toks[:70], 0)
        m.prefill(toks, 0, 32)
        m.prefill(toks, 32, 32)
        m.prefill(toks, 64, 6)
        for i in range(70, 75):
            a = m.forward(int(toks[i]), i)
            b = c2.forward(int(toks[i]), i)
            assert float(np.max(np.abs(a - b))) <= 1e-2 * rms(a), (dim, heads, kv, i)
        for wv in (False, True):
            d = kv_quant_diff(c2.copy_kv(0, wv), m.kv(0, wv), m, 75)
            assert d.max() <= 1 and d.mean() < 0.01, (dim, heads, kv, wv, int(d.max()), float(d.mean()))
        m.close()


def test_prefill_split_k_residual(torch_gpu, cpuref):
    """A prompt pass whose down projection (K = 2048 over 4 output tiles) runs
    as a split-K GEMM adding into the residual rows through the split
    reduction: the logits of the next steps within the full-model
    tolerance."""
    g = synth.synthetic_model(arch="llama", dim=256, hidden=2048, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128,
                              qtype=synth.Q8_0, seed=41, norm_jitter=0.1)
    toks = np.random.default_rng(41).integers(0, 512, 45).astype(np.int32)
    with l3p.Context(0) as c2:
        c2.load_gguf(g)
        m = cpuref.open_model(g)
        c2.prefill(toks[:40], 0)
        m.prefill(toks, 0, 40)
        for i in range(40, 45):
            a = m.forward(int(toks[i]), i)
            b = c2.forward(int(toks[i]), i)
            assert float(np.max(np.abs(a - b))) <= 1e-2 * rms(a), i
        m.close()


PATH_CASES = {
    # head size 64 (60-position chunks), 1400 positions: 24 chunks, 2 per wave for most waves
    "llama_hs64": (dict(arch="llama", dim=512, hidden=512, n_layers=3, n_heads=8, n_kv=2, vocab=512, ctx=2048,
                        qtype=synth.Q8_0, seed=31, norm_jitter=0.1), 1400),
    # head size 96 (40-position chunks, three blocks per row), odd group size
    "llama_hs96": (dict(arch="llama", dim=768, hidden=512, n_layers=2, n_heads=8, n_kv=4, vocab=512, ctx=1024,
                        qtype=synth.Q8_0, seed=32, norm_jitter=0.1), 700),
    # head size 256 (15-position chunks), QK-norm, NEOX RoPE, a sliding window
    # of 101 positions on five of six layers
    "gemma_hs256": (dict(arch="gemma3", dim=512, hidden=512, n_layers=6, n_heads=4, n_kv=2, head_dim=256, vocab=512,
                         ctx=1024, qtype=synth.Q8_0, seed=33, softcap=30.0, swa_window=101, norm_jitter=0.1,
                         tied=True), 600),
    # head size 128 (136-byte rows): windows starting at odd positions put the
    # first row 8 bytes into a 16-byte piece
    "gemma_hs128": (dict(arch="gemma3", dim=512, hidden=512, n_layers=6, n_heads=8, n_kv=2, head_dim=128, vocab=512,
                         ctx=1024, qtype=synth.Q8_0, seed=34, softcap=30.0, swa_window=101, norm_jitter=0.1,
                         tied=True), 600),
    # more than 64 chunks of 64 positions (4300 positions: 68 chunks), so the
    # chunk merge takes two rounds
    "llama_long": (dict(arch="llama", dim=256, hidden=256, n_layers=2, n_heads=4, n_kv=2, vocab=512, ctx=4608,
                        qtype=synth.Q8_0, seed=35, norm_jitter=0.1), 4300),
}


def test_wide_gemv_matches_chunk_columns(torch_gpu, cpuref, monkeypatch):
    """Gemma-2-2B widths: the decode step's Q8_0 GEMVs over 2304 columns
    (q|k|v and gate|up with the fused post-norm update, the LM head with the
    last post norm and the final norm) stream whole rows per wave by default
    (gemv_wide_kernel); L3P_GEMV_WIDE=0 takes the chunk-column kernel.  Each
    context captures its step graph with its own setting.  The two kernels
    sum every row in another order, so logits agree to 1e-3 * rms and the
    K/V caches within one quant step; against the oracle the whole-row
    logits are within the full-model tolerance, with the same greedy token
    wherever the oracle's top-2 margin is clear of it."""
    g = synth.synthetic_model(arch="gemma3", dim=2304, hidden=9216, n_layers=3, n_heads=8, n_kv=4, head_dim=256,
                              vocab=2048, ctx=64, qtype=synth.Q8_0, seed=31, softcap=30.0, swa_window=16,
                              norm_jitter=0.1, tied=True)
    toks = np.random.default_rng(31).integers(0, 2048, 12).astype(np.int32)
    m = cpuref.open_model(g)
    with l3p.Context(0) as cw, l3p.Context(0) as cc:
        for c, wide in ((cw, "1"), (cc, "0")):
            monkeypatch.setenv("L3P_GEMV_WIDE", wide)
            c.load_gguf(g)
            c.prefill(toks[:8], 0)
            c.forward(int(toks[8]), 8)   # captures the step graph with this setting
        monkeypatch.delenv("L3P_GEMV_WIDE", raising=False)
        m.prefill(toks[:8], 0, 8)
        m.forward(int(toks[8]), 8)
        tok = int(toks[9])
        for pos in range(9, 13):
            a = cw.forward(tok, pos)
            b = cc.forward(tok, pos)
            r = m.forward(tok, pos)
            assert float(np.max(np.abs(a - b))) <= 1e-3 * rms(b), pos
            assert float(np.max(np.abs(a - r))) <= 1e-2 * rms(r), pos
            if margin(r) > 2e-2 * rms(r):
                assert int(np.argmax(a)) == int(np.argmax(r)), pos
            tok = int(np.argmax(r))
        for layer in range(m.n_layers):
            for wv in (False, True):
                d = kv_quant_diff(cw.copy_kv(layer, wv), cc.copy_kv(layer, wv), m, 13)
                assert d.max() <= 1, (layer, wv, int(d.max()))
    m.close()


@pytest.mark.parametrize("case", list(PATH_CASES))
def test_prompt_attention_paths_agree(torch_gpu, monkeypatch, case):
    """A prompt through attn_prefill_kernel (the default) and through chunks +
    merge over a token grid dimension (L3P_PREFILL_ATTN=chunks): both score
    with the same exact Q8_0 block dots and differ only in the softmax and V
    summation order, so the layer-0 cache (written before any attention) is
    identical, deeper layers differ by at most one-step quant flips, and the
    next step's logits agree to 1e-2 * rms, the full-model tolerance after a
    prompt (each layer's difference reaches the K/V rows of every position of
    the next).  The cases cover head sizes 64 to 256, GQA groups of 2 and 4,
    sliding windows and 4300 positions."""
    kw, n_prompt = PATH_CASES[case]
    g = synth.synthetic_model(**kw)
    toks = np.random.default_rng(kw["seed"] + 1).integers(0, kw["vocab"], n_prompt + 1).astype(np.int32)
    with l3p.Context(0) as cf, l3p.Context(0) as cc:
        for c, path in ((cf, None), (cc, "chunks")):
            if path:
                monkeypatch.setenv("L3P_PREFILL_ATTN", path)
            else:
                monkeypatch.delenv("L3P_PREFILL_ATTN", raising=False)
            c.load_gguf(g)
            c.prefill(toks[:n_prompt], 0)
        monkeypatch.delenv("L3P_PREFILL_ATTN", raising=False)
        a = cf.forward(int(toks[n_prompt]), n_prompt)
        b = cc.forward(int(toks[n_prompt]), n_prompt)
        assert float(np.max(np.abs(a - b))) <= 1e-2 * rms(b), case
        mi = cf.model_info()
        for wv in (False, True):
            assert np.array_equal(cf.copy_kv(0, wv), cc.copy_kv(0, wv)), (case, wv)
            for layer in range(1, mi.n_layers):
                qa = cf.copy_kv(layer, wv).reshape(mi.n_kv_heads, mi.seq_len, -1, 34)[:, :n_prompt + 1, :, 2:]
                qb = cc.copy_kv(layer, wv).reshape(mi.n_kv_heads, mi.seq_len, -1, 34)[:, :n_prompt + 1, :, 2:]
                d = np.abs(qa.view(np.int8).astype(np.int32) - qb.view(np.int8).astype(np.int32))
                assert d.max() <= 1, (case, layer, wv, int(d.max()))


@pytest.mark.parametrize("case", list(PATH_CASES))
def test_attention_paths_agree(torch_gpu, monkeypatch, case):
    """The two decode attentions give the same steps: one workgroup per query
    head (L3P_ATTN_HEAD=1; by default for steps attending to fewer than 448
    positions, 192 at head_dim >= 192) and split position chunks with a merge
    kernel (L3P_ATTN_HEAD=0; by default from there on).  Both form the
    step's K/V rows with the same arithmetic, so the layer-0 cache (whose
    inputs are the embeddings) is bit-identical and deeper layers differ by
    at most one-step quant flips; the attention outputs differ only in fp32
    summation order, so logits agree to 1e-3 * rms.  Every wave of the
    per-head kernel takes one or more chunks at these lengths."""
    kw, n_prompt = PATH_CASES[case]
    g = synth.synthetic_model(**kw)
    rng = np.random.default_rng(kw["seed"])
    toks = rng.integers(0, kw["vocab"], n_prompt + 6).astype(np.int32)
    with l3p.Context(0) as ch, l3p.Context(0) as cc:
        for c in (ch, cc):
            c.load_gguf(g)
            c.prefill(toks[:n_prompt], 0)
        for i in range(n_prompt, n_prompt + 6):
            monkeypatch.setenv("L3P_ATTN_HEAD", "1")
            a = ch.forward(int(toks[i]), i)
            monkeypatch.setenv("L3P_ATTN_HEAD", "0")
            b = cc.forward(int(toks[i]), i)
            assert float(np.max(np.abs(a - b))) <= 1e-3 * rms(b), (case, i)
        mi = ch.model_info()
        for wv in (False, True):
            ka, kb = ch.copy_kv(0, wv), cc.copy_kv(0, wv)
            assert np.array_equal(ka, kb), (case, wv)
            for layer in range(1, mi.n_layers):
                qa = ch.copy_kv(layer, wv).reshape(mi.n_kv_heads, mi.seq_len, -1, 34)[:, :n_prompt + 6, :, 2:]
                qb = cc.copy_kv(layer, wv).reshape(mi.n_kv_heads, mi.seq_len, -1, 34)[:, :n_prompt + 6, :, 2:]
                d = np.abs(qa.view(np.int8).astype(np.int32) - qb.view(np.int8).astype(np.int32))
                assert d.max() <= 1, (case, layer, wv, int(d.max()))


@pytest.mark.parametrize("cap", [0.0, 0.3])
def test_attention_overrides_match_oracle(ctx, cpuref, monkeypatch, cap):
    """The load options without a counterpart in the reference: Gemma-2's
    alternating sliding-window layers (swa_pattern 2: layers 0, 2, 4, 6
    local, the rest global) and its attention score cap cap * tanh(s / cap)
    (the oracle's capped attention is pinned to that closed form in
    test_oracle_primitives).  A 7-layer Gemma with a 16-position window: a
    prefilled 40-token prompt, then 12 teacher-forced steps, the first six
    on the per-head kernel and the rest on chunks + merge, against the
    oracle with the same options; and the options must change the logits.
    Scores of this random model stay within about 1, so a cap of 0.3 bites."""
    kw = dict(MODELS["gemma_q8_0"])
    g = synth.synthetic_model(**kw)
    m = cpuref.open_model(g)
    m.set_attention(2, cap)
    ctx.load_gguf(g, swa_pattern=2, attn_softcap=cap)
    mi = ctx.model_info()
    assert mi.swa_pattern == 2 and abs(mi.attn_softcap - cap) < 1e-7
    prompt = np.random.default_rng(11).integers(0, m.vocab, 41).astype(np.int32)
    ctx.prefill(prompt[:-1], 0)
    m.prefill(prompt[:-1], 0, len(prompt) - 1)
    tok, pos = int(prompt[-1]), len(prompt) - 1
    logits = []
    for step in range(12):
        monkeypatch.setenv("L3P_ATTN_HEAD", "1" if step < 6 else "0")
        lo_ref = m.forward(tok, pos)
        lo_gpu = ctx.forward(tok, pos)
        tol = max(1e-2, 2.0 * REF_DRIFT["gemma_q8_0"]["max_rel"]) * rms(lo_ref)
        err = float(np.max(np.abs(lo_gpu - lo_ref)))
        assert err <= tol, f"step {step}: max |dlogit| {err:.3g} > {tol:.3g}"
        logits.append(lo_ref)
        tok, pos = int(np.argmax(lo_ref)), pos + 1
    monkeypatch.delenv("L3P_ATTN_HEAD", raising=False)
    m.close()
    # the same steps without the options differ by far more than the tolerance
    m0 = cpuref.open_model(g)
    m0.prefill(prompt[:-1], 0, len(prompt) - 1)
    tok, pos, moved = int(prompt[-1]), len(prompt) - 1, 0.0
    for step in range(12):
        lo = m0.forward(tok, pos)
        moved = max(moved, float(np.max(np.abs(lo - logits[step]))) / rms(lo))
        tok, pos = int(np.argmax(logits[step])), pos + 1
    m0.close()
    assert moved > 0.05, moved
