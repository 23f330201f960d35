"""l3p_gemm_static: the allocation-free l3p_gemm (file-scope split-K
partials, no context), called through the C-ABI, against l3p_gemm on the same
inputs: bit-identical outputs (the same kernels and the same launch plan), on
two calls in a row, the second smaller, both cutting K over several
workgroups (stream-K) so the file-scope partials are used; the same call captured into a HIP graph and replayed; a
shape whose partials exceed the array is rejected without a launch."""
import ctypes as C

import numpy as np
import pytest

import llama3pure_amd as l3p
from llama3pure_amd import synth

pytestmark = pytest.mark.gpu


def _static(L, qt, w, rows, cols, x, batch, y, stream):
    return L.l3p_gemm_static(qt, w.data_ptr(), rows, cols, x.data_ptr(), batch, cols, y.data_ptr(), rows, stream)


@pytest.mark.parametrize("qt", [synth.Q8_0, synth.Q4_K, synth.Q4_0])
def test_gemm_static_equals_gemm(torch_gpu, qt):
    torch = torch_gpu
    L = l3p.lib()
    with l3p.Context(0) as ctx:
        # rows x cols x batch: 64 output tiles of one 64-row tile whose K is
        # cut over 8 workgroups each (partials of 8 x 8 x 4096 floats), then a
        # smaller call cut over 4; Q4_0 takes the int8 path with its quantized
        # activation rows in the array
        for rows, cols, batch in ((4096, 4096, 8), (1024, 2048, 3)):
            w = torch.from_numpy(synth.random_blocks(qt, rows, cols, seed=rows + batch)).cuda()
            x = torch.from_numpy(synth.random_x(cols, seed=cols, batch=batch)).cuda()
            y_ref = torch.full((batch, rows), float("nan"), device="cuda")
            y_st = torch.full((batch, rows), float("nan"), device="cuda")
            torch.cuda.synchronize()
            ctx.gemm(qt, w, rows, cols, x, batch, cols, y_ref, rows)
            ctx.synchronize()
            rc = _static(L, qt, w, rows, cols, x, batch, y_st, ctx.stream)
            assert rc == l3p.OK, L.l3p_last_error(None).decode()
            ctx.synchronize()
            a, b = y_ref.cpu().numpy(), y_st.cpu().numpy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (qt, rows, cols, batch)


@pytest.mark.parametrize("qt", [synth.Q8_0, synth.Q4_0])
def test_gemm_static_in_graph(torch_gpu, qt):
    """For callers under graph capture: after one warm call (which looks up
    the array's address and the launch plan), l3p_gemm_static is captured on
    a stream into a graph; every replay, with eager work and synchronizations
    between replays, equals l3p_gemm bit for bit.  4096 x 4096 x batch 8
    cuts K over 8 workgroups per tile (Q8_0), so the replays use the
    file-scope partials; Q4_0 keeps its quantized activation rows there."""
    torch = torch_gpu
    L = l3p.lib()
    rows, cols, batch = 4096, 4096, 8
    with l3p.Context(0) as ctx:
        w = torch.from_numpy(synth.random_blocks(qt, rows, cols, seed=11)).cuda()
        x = torch.from_numpy(synth.random_x(cols, seed=12, batch=batch)).cuda()
        y_ref = torch.full((batch, rows), float("nan"), device="cuda")
        y_st = torch.full((batch, rows), float("nan"), device="cuda")
        torch.cuda.synchronize()
        ctx.gemm(qt, w, rows, cols, x, batch, cols, y_ref, rows)
        ctx.synchronize()
        ref = y_ref.cpu().numpy().view(np.uint32)
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            assert _static(L, qt, w, rows, cols, x, batch, y_st, s.cuda_stream) == l3p.OK   # warm
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            rc = _static(L, qt, w, rows, cols, x, batch, y_st, s.cuda_stream)
        assert rc == l3p.OK, L.l3p_last_error(None).decode()
        for rep in range(3):
            y_st.fill_(float("nan"))
            x.mul_(1.0)                 # eager work on the inputs between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(y_st.cpu().numpy().view(np.uint32), ref), (qt, rep)


def test_gemm_static_rejects_oversized_partials(torch_gpu):
    torch = torch_gpu
    L = l3p.lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    # T x 3 output tiles of 64 x 64 with 3 T below four workgroups per CU (so
    # the plan cuts K over at least two workgroups per tile of 16 K steps):
    # at least 2 x 192 x 64 T floats of partials, more than the 4 Mi of the
    # file-scope array once T > 170
    tiles = min(341, (4 * cus + 2) // 3 - 1)
    if tiles <= 171:
        pytest.skip(f"{cus} CUs: no shape of this form splits with partials past the array")
    with l3p.Context(0) as ctx:
        rows, cols, batch = 64 * tiles, 1024, 192
        w = torch.zeros(rows * synth.row_bytes(synth.Q8_0, cols), dtype=torch.uint8, device="cuda")
        x = torch.zeros(batch * cols, device="cuda")
        y = torch.zeros(batch * rows, device="cuda")
        torch.cuda.synchronize()
        rc = L.l3p_gemm_static(synth.Q8_0, w.data_ptr(), rows, cols, x.data_ptr(), batch, cols, y.data_ptr(), rows,
                               ctx.stream)
        assert rc == l3p.E_UNSUPPORTED
        assert b"static scratch" in L.l3p_last_error(None)
        # bad arguments are rejected before anything runs
        assert L.l3p_gemm_static(synth.Q8_0, w.data_ptr(), -1, cols, x.data_ptr(), 1, cols, y.data_ptr(), rows,
                                 ctx.stream) == l3p.E_INVALID
        assert L.l3p_gemm_static(synth.Q8_0, w.data_ptr(), rows, 0, x.data_ptr(), 1, cols, y.data_ptr(), rows,
                                 ctx.stream) == l3p.E_INVALID


def test_gemm_static_q8_activation_chunks(torch_gpu):
    """Q4_0 rows whose quantized form exceeds the file-scope array go through
    it in several launches (1000 rows of 14336 columns: 4480 floats a row
    against 4 Mi floats); each output adds its blocks in order whatever the
    rows per launch, so the result equals l3p_gemm's (one launch) bit for
    bit."""
    torch = torch_gpu
    L = l3p.lib()
    rows, cols, batch = 256, 14336, 1000
    with l3p.Context(0) as ctx:
        w = torch.from_numpy(synth.random_blocks(synth.Q4_0, rows, cols, seed=21)).cuda()
        x = torch.from_numpy(synth.random_x(cols, seed=22, batch=batch)).cuda()
        y_ref = torch.full((batch, rows), float("nan"), device="cuda")
        y_st = torch.full((batch, rows), float("nan"), device="cuda")
        torch.cuda.synchronize()
        ctx.gemm(synth.Q4_0, w, rows, cols, x, batch, cols, y_ref, rows)
        ctx.synchronize()
        rc = _static(L, synth.Q4_0, w, rows, cols, x, batch, y_st, ctx.stream)
        assert rc == l3p.OK, L.l3p_last_error(None).decode()
        ctx.synchronize()
        assert np.array_equal(y_ref.cpu().numpy().view(np.uint32), y_st.cpu().numpy().view(np.uint32))
