"""Error paths of the C-ABI (through ctypes): malformed GGUF images, shapes
and ranges the entry points refuse, and calls out of order.  Every refusal
is an L3P_E_* code with a message; the context stays usable afterwards.

The reference's behaviour on the same inputs: a bad magic or version, a
truncated file or an unsupported tensor type ends the C engine with exit(1)
(c:2515-2537, c:2123-2124) and makes the JS engine throw into llama3pure()'s
try/catch (js:4129-4134, js:7246-7248); here each is a return code."""
import struct

import numpy as np
import pytest

import llama3pure_amd as l3p
from llama3pure_amd import synth

pytestmark = pytest.mark.gpu

SMALL = dict(arch="llama", dim=256, hidden=256, n_layers=2, n_heads=4, n_kv=2, vocab=256, ctx=128,
             qtype=synth.Q8_0, seed=61)


@pytest.fixture(scope="module")
def good():
    return synth.synthetic_model(**SMALL)


def load_err(ctx, img, **kw):
    with pytest.raises(l3p.L3PError) as e:
        ctx.load_gguf(img, **kw)
    return e.value


def test_bad_magic_and_version(ctx, good):
    e = load_err(ctx, b"GGUX" + good[4:])
    assert e.code == l3p.E_FORMAT and "magic" in str(e)
    for ver in (1, 4):
        e = load_err(ctx, good[:4] + struct.pack("<I", ver) + good[8:])
        assert e.code == l3p.E_FORMAT and "version" in str(e), ver


@pytest.mark.parametrize("cut", [0, 10, 23, 100, 2000, -1])
def test_truncated(ctx, good, cut):
    """Cut in the header, the metadata, the tensor infos and the last tensor's data."""
    n = len(good) + cut if cut < 0 else cut
    e = load_err(ctx, good[:n])
    assert e.code == l3p.E_FORMAT, (cut, str(e))


def test_unsupported_tensor_type(ctx):
    """A tensor of a GGML type the reference has no kernel for (16, IQ2_XXS)."""
    meta = {"general.architecture": "llama", "llama.embedding_length": 256, "llama.block_count": 1}
    img = synth.write_gguf(meta, [("token_embd.weight", 16, (256, 4), bytes(4 * 66))])
    e = load_err(ctx, img)
    assert e.code == l3p.E_UNSUPPORTED and "type" in str(e)


def test_missing_tensor(ctx, good):
    meta = {"general.architecture": "llama", "llama.embedding_length": 256, "llama.block_count": 1,
            "llama.attention.head_count": 4, "llama.vocab_size": 4}
    img = synth.write_gguf(meta, [("token_embd.weight", synth.Q8_0, (256, 4), bytes(4 * 272))])
    e = load_err(ctx, img)
    assert e.code == l3p.E_FORMAT and "not found" in str(e)


def test_context_option(ctx, good):
    """A context_size option above the model's context is ignored, as in the
    reference (c:5174-5178); one below it shortens the KV cache."""
    assert ctx.load_gguf(good, context_size=100000).seq_len == SMALL["ctx"]
    assert ctx.load_gguf(good, context_size=64).seq_len == 64
    with pytest.raises(l3p.L3PError) as e:
        ctx.forward(1, 64)                            # past the shortened context
    assert e.value.code == l3p.E_INVALID


def test_attention_option_ranges(ctx, good):
    """swa_pattern and attn_softcap (options without a counterpart in the
    reference) must be finite and not negative: a negative value, an infinite
    cap (cap * tanh(s / cap) would be inf * 0 = NaN for every score) and a NaN
    cap are refused with L3P_E_INVALID, and the context then loads normally."""
    for opts in (dict(swa_pattern=-1), dict(attn_softcap=-1.0), dict(attn_softcap=float("inf")),
                 dict(attn_softcap=float("nan"))):
        with pytest.raises(l3p.L3PError) as e:
            ctx.load_gguf(good, **opts)
        assert e.value.code == l3p.E_INVALID, opts
    assert ctx.load_gguf(good, attn_softcap=50.0).attn_softcap == 50.0


def test_out_of_memory_context(torch_gpu):
    """A context whose K/V cache cannot fit the GPU (40 layers x 64 KV heads
    of 256 x 262144 positions: 365 GB) fails with L3P_E_NOMEM after freeing
    what it allocated, and the context then loads a model normally."""
    def zeros(qtype, rows, cols, std, view):
        view[:] = 0
        return view
    big = synth.synthetic_model(arch="llama", dim=256, hidden=256, n_layers=40, n_heads=64, n_kv=64, head_dim=256,
                                vocab=64, ctx=262144, qtype=synth.Q8_0, seed=62, make_mat=zeros)
    with l3p.Context(0) as c:
        free0 = torch_gpu.cuda.mem_get_info()[0]
        with pytest.raises(l3p.L3PError) as e:
            c.load_gguf(big)
        assert e.value.code == l3p.E_NOMEM, str(e.value)
        assert torch_gpu.cuda.mem_get_info()[0] >= free0 - (256 << 20)   # nothing left behind
        assert c.load_gguf(synth.synthetic_model(**SMALL)).n_layers == 2
        c.forward(3, 0)


def test_calls_out_of_order_and_ranges(torch_gpu, good):
    with l3p.Context(0) as c:
        with pytest.raises(l3p.L3PError) as e:
            c.forward(1, 0)                           # no model loaded
        assert e.value.code == l3p.E_STATE
        c.load_gguf(good)
        for tok, pos in ((-1, 0), (SMALL["vocab"], 0), (1, -1), (1, SMALL["ctx"])):
            with pytest.raises(l3p.L3PError) as e:
                c.forward(tok, pos)
            assert e.value.code == l3p.E_INVALID, (tok, pos)
        toks = np.arange(4, dtype=np.int32)
        # start + n would overflow a 32-bit int: refused, nothing written
        L = l3p.lib()
        for start, n in ((2**31 - 2, 4), (SMALL["ctx"] - 2, 4), (-1, 4)):
            assert L.l3p_prefill(c.h, toks.ctypes.data, n, start) == l3p.E_INVALID, (start, n)
        assert L.l3p_prefill(c.h, toks.ctypes.data, -1, 0) == l3p.E_INVALID
        with pytest.raises(l3p.L3PError) as e:
            c.prefill(np.array([0, SMALL["vocab"]], np.int32), 0)   # token out of range
        assert e.value.code == l3p.E_INVALID


def test_gemm_shape_checks(ctx, torch_gpu):
    x = torch_gpu.zeros(4 * 512, device="cuda")
    y = torch_gpu.zeros(4 * 512, device="cuda")
    w = torch_gpu.zeros(512 * 544, dtype=torch_gpu.uint8, device="cuda")
    for rows, cols in ((-1, 512), (512, 0), (512, -32), (512, 500)):
        with pytest.raises(l3p.L3PError) as e:
            ctx.gemm(l3p.Q8_0, w, rows, cols, x, 4, 512, y, 512)
        assert e.value.code == l3p.E_INVALID, (rows, cols)
    with pytest.raises(l3p.L3PError) as e:
        ctx.gemm(l3p.Q8_0, w, 512, 512, x, -1, 512, y, 512)
    assert e.value.code == l3p.E_INVALID
