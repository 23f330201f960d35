"""GPU parity of the standalone ops, through the C-ABI (libl3p.so).

Bit-exact: dequantization and the Q8_0 quantizer.  GEMV: within the stated
fp32 summation tolerance of the float64 value of the reference arithmetic:

    |y_gpu - y64| <= gamma_(K+4) * S,   gamma_n = n u / (1 - n u), u = 2^-24

where S bounds the magnitudes summed by either side:
    Q8_0, F16, BF16:  S = sum_j |w_j x_j|
    Q4_0, Q4_1, Q5_0, Q5_1, IQ4_NL:
           S = sum_blocks |dw dx isum| (+ |mw dx xsum|)   (integer block dots are exact)
    Q2_K, Q4_K, Q5_K:
           S = sum_j (|d1 q_j| + |m1|) |x_j|   (the Q4_K and Q5_K kernels factor scale and min out of a group)
    Q3_K:  S = sum_j |d s| (v_j + 4) |x_j|     (code v in 0..7, offset 4)
    Q6_K:  S = sum_j |d sc| (|q_j| + 32) |x_j| (kernel factors d sc, offset 32)
and the oracle itself must satisfy the same bound.
"""
import numpy as np
import pytest

import llama3pure_amd as l3p
import oracle
from block_math import kquant_magnitudes, q8_block_terms
from llama3pure_amd import synth

pytestmark = pytest.mark.gpu


def gamma(n):
    u = 2.0 ** -24
    return n * u / (1 - n * u)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def empty_f32(torch, n):
    return torch.empty(n, dtype=torch.float32, device="cuda")


# --------------------------------------------------------------------------- dequant / quantize
@pytest.mark.parametrize("qtype", [l3p.Q8_0, l3p.Q4_0, l3p.Q4_1, l3p.Q5_0, l3p.Q5_1, l3p.Q2_K, l3p.Q3_K, l3p.Q4_K,
                                   l3p.Q5_K, l3p.Q6_K, l3p.IQ4_NL, l3p.F16, l3p.BF16, l3p.F32])
def test_dequant_bit_exact(ctx, torch_gpu, cpuref, qtype):
    e, bb = oracle.BLOCK[qtype]
    n = 256 * 40
    raw = np.random.default_rng(qtype + 100).integers(0, 256, n // e * bb, dtype=np.uint8)
    if qtype in (l3p.Q8_0, l3p.Q4_0, l3p.Q4_K, l3p.Q6_K):
        raw[: synth.row_bytes(qtype, 2048)] = synth.random_blocks(qtype, 1, 2048, seed=3)[0]
    d = dev(torch_gpu, raw)
    out = empty_f32(torch_gpu, n)
    ctx.dequant(qtype, d, n, out)
    ctx.synchronize()
    want = cpuref.dequant(qtype, raw, n)
    got = out.cpu().numpy()
    # random bytes include NaN fp16 scales: NaN outputs must match in place;
    # their payload and sign (which the CPU and GPU propagate differently
    # through a - b) are not compared
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_quantize_q8_0_bit_exact(ctx, torch_gpu, cpuref):
    rng = np.random.default_rng(7)
    n = 32 * 4096
    x = (rng.standard_normal(n) * np.float32(10.0) ** rng.integers(-8, 5, n)).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = np.array([127.0] + [k + 0.5 for k in range(-15, 16)], np.float32)   # exact .5 ties
    x[64:96] = 1e-30                                                               # subnormal scale
    x[96:128] = -np.float32(3.0e38)
    out = torch_gpu.empty(n // 32 * 34, dtype=torch_gpu.uint8, device="cuda")
    ctx.quantize_q8_0(dev(torch_gpu, x), n, out)
    ctx.synchronize()
    assert np.array_equal(out.cpu().numpy(), cpuref.quantize_q8_0(x))


# --------------------------------------------------------------------------- GEMV
Q8_ACT = (l3p.Q4_0, l3p.Q4_1, l3p.Q5_0, l3p.Q5_1, l3p.IQ4_NL)
K_QUANTS = (l3p.Q2_K, l3p.Q3_K, l3p.Q4_K, l3p.Q5_K, l3p.Q6_K)


def _bound_terms(cpuref, qtype, w, rows, cols, x):
    """(y64, S) of the reference arithmetic in float64, per the module doc."""
    x64 = x.astype(np.float64)
    if qtype in Q8_ACT:
        terms = q8_block_terms(cpuref, qtype, w, rows, cols, x)
        return terms.sum(1), np.abs(terms).sum(1)
    W = np.stack([cpuref.dequant(qtype, w[r], cols) for r in range(rows)]).astype(np.float64)
    y64 = W @ x64
    if qtype in K_QUANTS:
        return y64, kquant_magnitudes(qtype, w, rows, cols) @ np.abs(x64)
    return y64, np.abs(W) @ np.abs(x64)


def _check_gemv(ctx, torch, cpuref, qtype, rows, cols, seed=0, sample_rows=None):
    w = synth.random_blocks(qtype, rows, cols, seed=seed)
    x = synth.random_x(cols, seed=seed + 1)
    y = empty_f32(torch, rows)
    ctx.gemv(qtype, dev(torch, w), rows, cols, dev(torch, x), y)
    ctx.synchronize()
    got = y.cpu().numpy()
    idx = np.arange(rows) if sample_rows is None else np.random.default_rng(seed).choice(rows, sample_rows, False)
    wi = w[idx]
    y64, S = _bound_terms(cpuref, qtype, wi, len(idx), cols, x)
    tol = gamma(cols + 4) * S
    ref = cpuref.matmul(qtype, wi, len(idx), cols, x)
    assert np.all(np.abs(ref - y64) <= tol), "oracle outside its own bound"
    err = np.abs(got[idx] - y64)
    assert np.all(err <= tol), f"max err/tol {np.max(err / np.maximum(tol, 1e-30)):.3g}"
    return got


@pytest.mark.parametrize("qtype,rows,cols", [
    (l3p.Q8_0, 4096, 4096),        # attention shape
    (l3p.Q8_0, 1024, 14336),
    (l3p.Q4_0, 14336, 4096),       # FFN gate/up
    (l3p.Q4_0, 4096, 14336),       # FFN down
    (l3p.Q4_K, 14336, 4096),
    (l3p.Q6_K, 2048, 4096),
    (l3p.Q8_0, 2304, 2304),        # Gemma-2-2B dims
    (l3p.Q8_0, 2304, 9216),
    (l3p.Q4_0, 2304, 2304),        # last column chunk of 8 blocks
    (l3p.Q4_0, 1000, 9216),
    (l3p.Q8_0, 300, 256),          # one partial chunk
    (l3p.Q4_0, 77, 1536),
    (l3p.Q8_0, 128256 // 64, 4096),
    # rows that are not 16-byte multiples (copied from 16-byte aligned-down
    # addresses): Gemma-3-1B / 270M widths, tiny rows, Q6_K off 2048-multiples
    (l3p.Q8_0, 2048, 1152),
    (l3p.Q8_0, 1025, 640),
    (l3p.Q8_0, 99, 96),
    (l3p.Q4_0, 2048, 1152),
    (l3p.Q4_0, 333, 160),
    (l3p.Q6_K, 1000, 2304),
    (l3p.Q6_K, 512, 1536),
    (l3p.Q6_K, 301, 256),
    (l3p.Q6_K, 4097, 14336),
    # Q4_K: partial last chunk (9 super-blocks), one super-block, FFN down
    (l3p.Q4_K, 2304, 2304),
    (l3p.Q4_K, 100, 256),
    (l3p.Q4_K, 4096, 14336),
    # the other types: a full-width shape, a partial last chunk, and rows
    # that are not 16-byte multiples where the type allows them
    (l3p.Q4_1, 2048, 4096),
    (l3p.Q4_1, 700, 1120),         # 700 B rows
    (l3p.Q5_0, 2048, 4096),
    (l3p.Q5_0, 999, 1152),         # 792 B rows
    (l3p.Q5_1, 1024, 14336),
    (l3p.Q5_1, 515, 1120),         # 840 B rows
    (l3p.IQ4_NL, 2048, 4096),
    (l3p.IQ4_NL, 333, 160),
    # widths that leave a short last chunk column: 4160 columns (64 + 64 + 2
    # blocks), 2304 (64 + 8), 6400 (3 x 64 + 8)
    (l3p.Q8_0, 100, 4160),
    # Q8_0 widths whose last chunk column holds 8, 16 or 32 lane slots: rows
    # per group G = 8 and 16 with a ragged last group, 16 lane slots, one wave
    # of 32, three waves + 8
    (l3p.Q8_0, 6150, 2304),
    (l3p.Q8_0, 12289, 2304),
    (l3p.Q8_0, 1001, 2560),
    (l3p.Q8_0, 777, 1024),
    (l3p.Q8_0, 500, 4352),
    (l3p.Q4_1, 300, 4160),
    (l3p.Q5_0, 200, 2304),
    (l3p.IQ4_NL, 257, 2304),
    (l3p.Q5_1, 300, 6400),
    (l3p.Q2_K, 2048, 4096),
    (l3p.Q2_K, 1000, 2304),        # 756 B rows
    (l3p.Q3_K, 2048, 4096),
    (l3p.Q3_K, 1000, 2304),        # 990 B rows
    (l3p.Q3_K, 301, 256),
    (l3p.Q5_K, 2048, 4096),
    (l3p.Q5_K, 777, 2304),
    (l3p.F16, 1024, 4096),
    (l3p.F16, 200, 9216),
    (l3p.F16, 64, 32768),          # 16 chunk columns: two buffers per wave
    (l3p.BF16, 1024, 4096),
    (l3p.BF16, 99, 288),
    (l3p.BF16, 65, 30720),
    (l3p.F32, 1024, 4096),
    (l3p.F32, 70, 16384),          # 8 chunk columns: two buffers per wave
    (l3p.F32, 33, 96),
])
def test_gemv_parity(ctx, torch_gpu, cpuref, qtype, rows, cols):
    _check_gemv(ctx, torch_gpu, cpuref, qtype, rows, cols, seed=rows + cols, sample_rows=min(rows, 768))


def test_gemv_q6_k_lm_head_shape(ctx, torch_gpu, cpuref):
    """Q6_K at the 128256 x 4096 output-projection shape (rows sampled)."""
    _check_gemv(ctx, torch_gpu, cpuref, l3p.Q6_K, 128256, 4096, seed=9, sample_rows=512)


@pytest.mark.parametrize("qtype", [l3p.Q8_0, l3p.Q4_0, l3p.Q5_1, l3p.IQ4_NL, l3p.Q3_K, l3p.Q4_K, l3p.Q6_K,
                                   l3p.BF16])
@pytest.mark.parametrize("rows", [1, 3, 5, 7, 9, 4097])
def test_gemv_ragged_rows(ctx, torch_gpu, cpuref, qtype, rows):
    cols = 2048 if qtype == l3p.Q6_K else 512
    _check_gemv(ctx, torch_gpu, cpuref, qtype, rows, cols, seed=rows)


@pytest.mark.parametrize("cols", [2304, 2560])
@pytest.mark.parametrize("rows", [1, 2, 3, 5, 7, 9, 4097])
def test_gemv_wide_rows_ragged(ctx, torch_gpu, cpuref, monkeypatch, rows, cols):
    """Q8_0 rows of 2304 and 2560 columns stream whole rows per wave
    (gemv_wide_kernel, four rows per group): ragged last groups against the
    oracle's bound, and the chunk-column kernel (L3P_GEMV_WIDE=0) on the
    same inputs within the same bound."""
    got = _check_gemv(ctx, torch_gpu, cpuref, l3p.Q8_0, rows, cols, seed=rows + cols)
    monkeypatch.setenv("L3P_GEMV_WIDE", "0")
    old = _check_gemv(ctx, torch_gpu, cpuref, l3p.Q8_0, rows, cols, seed=rows + cols)
    if rows > 4096:   # different summation orders: some of 4097 row totals differ in their last bits
        assert not np.array_equal(got, old), "both runs took the same kernel"


@pytest.mark.parametrize("cols", [4608, 6912, 9216])
@pytest.mark.parametrize("rows", [1, 3, 5, 769, 2304, 4097])
def test_gemv_sliced_rows(ctx, torch_gpu, cpuref, monkeypatch, rows, cols):
    """Q8_0 rows of 2, 3 and 4 x 2304 columns (Gemma-2-2B's down projection
    has 9216): that many waves a workgroup, each streaming a 2304-column slice
    of every row, the slices' totals added in order; rows dealt over the
    workgroups, ragged counts included, against the oracle's bound, and the
    chunk-column kernel (L3P_GEMV_SLICED=0) on the same inputs within the
    same bound."""
    got = _check_gemv(ctx, torch_gpu, cpuref, l3p.Q8_0, rows, cols, seed=rows + cols, sample_rows=min(rows, 768))
    monkeypatch.setenv("L3P_GEMV_SLICED", "0")
    old = _check_gemv(ctx, torch_gpu, cpuref, l3p.Q8_0, rows, cols, seed=rows + cols, sample_rows=min(rows, 768))
    if rows >= 2304:   # different summation orders: some row totals differ in their last bits
        assert not np.array_equal(got, old), "both runs took the same kernel"


def test_gemv_zero_rows_and_errors(ctx, torch_gpu):
    x = empty_f32(torch_gpu, 512)
    y = empty_f32(torch_gpu, 8)
    ctx.gemv(l3p.Q8_0, 0, 0, 512, x, y)              # no rows: nothing to do
    with pytest.raises(l3p.L3PError) as e:
        ctx.gemv(l3p.Q8_0, 0, 8, 500, x, y)          # cols not a block multiple
    assert e.value.code == l3p.E_INVALID
    with pytest.raises(l3p.L3PError) as e:
        ctx.gemv(l3p.F32, 0, 8, 32768, x, y)         # F32 rows wider than 16384
    assert e.value.code == l3p.E_UNSUPPORTED
    with pytest.raises(l3p.L3PError) as e:
        ctx.gemv(l3p.Q8_0, 0, 8, 512, x, y)          # null weight pointer
    assert e.value.code == l3p.E_INVALID


def test_gemv_deterministic(ctx, torch_gpu):
    rows, cols = 4096, 4096
    w = dev(torch_gpu, synth.random_blocks(l3p.Q8_0, rows, cols, seed=1))
    x = dev(torch_gpu, synth.random_x(cols, seed=2))
    y1, y2 = empty_f32(torch_gpu, rows), empty_f32(torch_gpu, rows)
    ctx.gemv(l3p.Q8_0, w, rows, cols, x, y1)
    ctx.gemv(l3p.Q8_0, w, rows, cols, x, y2)
    ctx.synchronize()
    assert torch_gpu.equal(y1, y2)


@pytest.mark.parametrize("qtype", Q8_ACT)
@pytest.mark.parametrize("rows,cols,batch", [(1024, 2048, 7), (300, 4096, 130), (77, 96, 65), (1, 32, 1), (70, 160, 3)])
def test_gemm_q8_activation_parity(ctx, torch_gpu, cpuref, qtype, rows, cols, batch):
    """Batches of the Q8_0-activation types on the int8 matrix cores against
    the reference's batched dot (matmul_quantized_batch, c:2305-2318: every
    row quantized to Q8_0, vec_dot_*_q8_0 per block).  The block dots are
    exact integers and each output adds its block terms in block order with
    the reference's expression and roundings (sum + dw * dx * isum, plus
    mw * dx * xsum), so the outputs equal the oracle's batched dot (the
    reference's arithmetic without contraction, as its -O3 build computes it)
    bit for bit; both also lie within gamma_(blocks+4) S of the float64
    value, S = sum of |block terms|.  96 columns give a K step of one block;
    65 and 130 rows leave ragged row tiles; one row of one block, and 70 x
    160 x 3, are the smallest cases."""
    w = synth.random_blocks(qtype, rows, cols, seed=5)
    xb = synth.random_x(cols, seed=6, batch=batch)
    y = empty_f32(torch_gpu, batch * rows)
    ctx.gemm(qtype, dev(torch_gpu, w), rows, cols, dev(torch_gpu, xb), batch, cols, y, rows)
    ctx.synchronize()
    got = y.cpu().numpy().reshape(batch, rows).astype(np.float64)
    terms = [q8_block_terms(cpuref, qtype, w, rows, cols, xb[b]) for b in range(batch)]
    y64 = np.stack([t.sum(1) for t in terms])
    S = np.stack([np.abs(t).sum(1) for t in terms])
    ref = cpuref.matmul_batch(qtype, w, rows, cols, xb).astype(np.float64)
    tol = gamma(cols // 32 + 4) * S
    assert np.all(np.abs(ref - y64) <= tol), "oracle outside gamma_(blocks+4) S"
    err = np.abs(got - y64)
    assert np.all(err <= tol), f"max err/tol {np.max(err / np.maximum(tol, 1e-30)):.3g}"
    diff = np.argwhere(got.astype(np.float32) != ref.astype(np.float32))
    assert diff.size == 0, f"{len(diff)} of {got.size} outputs differ from the oracle, first {tuple(diff[0])}"


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
def test_gemm_q4_0_c2_shapes_bit_exact(ctx, torch_gpu, cpuref, rows, cols):
    """Q4_0 batches at the C2 shapes (Llama-3-8B's FFN up and down), 16
    activation rows: the int8 matrix-core GEMM equals the oracle's batched dot
    (matmul_quantized_batch, c:2305-2318) bit for bit."""
    batch = 16
    w = synth.random_blocks(l3p.Q4_0, rows, cols, seed=rows + 3)
    xb = synth.random_x(cols, seed=cols + 4, batch=batch)
    y = empty_f32(torch_gpu, batch * rows)
    ctx.gemm(l3p.Q4_0, dev(torch_gpu, w), rows, cols, dev(torch_gpu, xb), batch, cols, y, rows)
    ctx.synchronize()
    got = y.cpu().numpy().reshape(batch, rows)
    ref = cpuref.matmul_batch(l3p.Q4_0, w, rows, cols, xb)
    diff = np.argwhere(got != ref)
    assert diff.size == 0, f"{len(diff)} of {got.size} outputs differ from the oracle, first {tuple(diff[0])}"


@pytest.mark.parametrize("qtype", Q8_ACT)
def test_gemm_q8_activation_close_to_gemv(ctx, torch_gpu, cpuref, qtype):
    """The batched and the single-row (GEMV) forms of these types agree
    within twice the module's bound."""
    rows, cols, batch = 1024, 2048, 5
    w = synth.random_blocks(qtype, rows, cols, seed=15)
    xb = synth.random_x(cols, seed=16, batch=batch)
    wd, xd = dev(torch_gpu, w), dev(torch_gpu, xb)
    y = empty_f32(torch_gpu, batch * rows)
    ctx.gemm(qtype, wd, rows, cols, xd, batch, cols, y, rows)
    ys = []
    for b in range(batch):
        yb = empty_f32(torch_gpu, rows)
        ctx.gemv(qtype, wd, rows, cols, xd[b], yb)
        ys.append(yb)
    ctx.synchronize()
    S = np.stack([np.abs(q8_block_terms(cpuref, qtype, w, rows, cols, xb[b])).sum(1) for b in range(batch)])
    diff = np.abs(y.view(batch, rows).cpu().numpy().astype(np.float64) -
                  torch_gpu.stack(ys).cpu().numpy().astype(np.float64))
    assert np.all(diff <= 2 * gamma(cols + 4) * S)


GEMM_TYPES = (l3p.F32, l3p.F16, l3p.BF16, l3p.Q8_0, l3p.Q2_K, l3p.Q3_K, l3p.Q4_K, l3p.Q5_K, l3p.Q6_K)


@pytest.mark.parametrize("qtype", GEMM_TYPES)
def test_gemm_weight_tiles_exact(ctx, torch_gpu, cpuref, qtype):
    """The GEMM's weight tiles bit for bit: with unit activation rows
    (x_b = e_b) every output is one product w[n][b] * 1 plus exact zeros, so
    y[b][n] must be the reference's dequantized weight (dequantize_row_*,
    c:611-934).  512 columns hold every element position of two
    super-blocks; 200 rows leave a ragged row tile."""
    rows, cols = 200, 512
    w = synth.random_blocks(qtype, rows, cols, seed=7)
    eye = np.eye(cols, dtype=np.float32)
    y = torch_gpu.full((cols * rows,), float("nan"), dtype=torch_gpu.float32, device="cuda")
    ctx.gemm(qtype, dev(torch_gpu, w), rows, cols, dev(torch_gpu, eye), cols, cols, y, rows)
    ctx.synchronize()
    got = y.cpu().numpy().reshape(cols, rows)
    want = np.stack([cpuref.dequant(qtype, w[r], cols) for r in range(rows)]).T   # the reference's values
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} outputs differ, first (b, n) {tuple(bad[0])}: {got[tuple(bad[0])]!r} vs " \
                          f"{want[tuple(bad[0])]!r}"


def _dequant_bound(cpuref, qtype, w, rows, cols):
    """(W, A): the exact dequantized weights in float64 and the per-element
    magnitudes whose products with |x| bound either side's fp32 sums (module
    doc; the GEMM forms the exact w = d1 q - m1, which A also bounds)."""
    W = np.stack([cpuref.dequant(qtype, w[r], cols) for r in range(rows)]).astype(np.float64)
    if qtype in K_QUANTS:
        return W, kquant_magnitudes(qtype, w, rows, cols)
    return W, np.abs(W)


@pytest.mark.parametrize("qtype,rows,cols,batch", [
    (l3p.Q8_0, 1024, 2048, 7),
    (l3p.Q8_0, 2304, 2304, 130),     # Gemma-2-2B projection, 3 ragged batch tiles
    (l3p.Q8_0, 300, 96, 65),         # K of one and a half 64-wide steps
    (l3p.Q8_0, 2048, 1152, 33),      # rows that are not 16-byte multiples
    (l3p.Q8_0, 77, 14336, 1),
    (l3p.Q4_K, 1000, 2304, 17),
    (l3p.Q6_K, 513, 1536, 40),
    (l3p.Q2_K, 300, 2304, 9),
    (l3p.Q3_K, 260, 1024, 66),
    (l3p.Q5_K, 1000, 2304, 17),
    (l3p.F16, 130, 320, 5),
    (l3p.BF16, 257, 2048, 64),
    (l3p.F32, 100, 512, 70),
    # jobs large enough for 64 x 128 tiles (eight waves): ragged N and M,
    # K-quant slices, rows that are not 16-byte multiples
    (l3p.Q8_0, 8200, 512, 1000),
    (l3p.Q4_K, 8192, 512, 1024),
    (l3p.Q6_K, 8320, 256, 1000),
])
def test_gemm_mfma_parity(ctx, torch_gpu, cpuref, qtype, rows, cols, batch):
    """MFMA GEMM against the float64 value of the reference's dequantize-then-
    fp32-dot (matmul_deq_batch_4row, c:2179-2273), every output within the
    fp32 summation bound gamma_(K+4) * S of the module doc."""
    seed = rows + cols + batch
    w = synth.random_blocks(qtype, rows, cols, seed=seed)
    xb = synth.random_x(cols, seed=seed + 1, batch=batch)
    ld_out = rows + 3                  # strided output rows
    y = torch_gpu.full((batch * ld_out,), float("nan"), dtype=torch_gpu.float32, device="cuda")
    ctx.gemm(qtype, dev(torch_gpu, w), rows, cols, dev(torch_gpu, xb), batch, cols, y, ld_out)
    ctx.synchronize()
    got = y.cpu().numpy().reshape(batch, ld_out)
    W, A = _dequant_bound(cpuref, qtype, w, rows, cols)
    x64 = xb.astype(np.float64)
    y64 = x64 @ W.T
    tol = gamma(cols + 4) * (np.abs(x64) @ A.T)
    err = np.abs(got[:, :rows] - y64)
    assert np.all(err <= tol), f"max err/tol {np.max(err / np.maximum(tol, 1e-30)):.3g}"
    assert np.all(np.isnan(got[:, rows:])), "wrote outside the output rows"


@pytest.mark.parametrize("env", [{"L3P_GEMM_SK_BN": "128"}, {"L3P_GEMM_SK_WPC": "2"},
                                 {"L3P_GEMM_SK_MIN": "16"}, {"L3P_GEMM_SK_BN": "128", "L3P_GEMM_SK_WPC": "2"}])
def test_gemm_stream_k_overrides(ctx, torch_gpu, cpuref, env, monkeypatch):
    """The stream-K plan overrides (128-wide tiles, workgroups per CU, the
    shortest run) change only the schedule: a Gemma-2-2B-like output
    projection (2304 x 2048, 130 rows: stream-K) stays within the fp32
    summation bound under each of them."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    qtype, rows, cols, batch = l3p.Q8_0, 2304, 2048, 130
    w = synth.random_blocks(qtype, rows, cols, seed=31)
    xb = synth.random_x(cols, seed=32, batch=batch)
    y = torch_gpu.full((batch * rows,), float("nan"), dtype=torch_gpu.float32, device="cuda")
    ctx.gemm(qtype, dev(torch_gpu, w), rows, cols, dev(torch_gpu, xb), batch, cols, y, rows)
    ctx.synchronize()
    got = y.cpu().numpy().reshape(batch, rows)
    W, A = _dequant_bound(cpuref, qtype, w, rows, cols)
    x64 = xb.astype(np.float64)
    err = np.abs(got - x64 @ W.T)
    tol = gamma(cols + 4) * (np.abs(x64) @ A.T)
    assert np.all(err <= tol), f"max err/tol {np.max(err / np.maximum(tol, 1e-30)):.3g}"


def test_gemm_mfma_equals_gemv_within_bound(ctx, torch_gpu, cpuref):
    """The batched and the single-row forms agree within the same bound."""
    qtype, rows, cols, batch = l3p.Q8_0, 4096, 4096, 5
    w = synth.random_blocks(qtype, rows, cols, seed=11)
    xb = synth.random_x(cols, seed=12, batch=batch)
    wd, xd = dev(torch_gpu, w), dev(torch_gpu, xb)
    y = empty_f32(torch_gpu, batch * rows)
    ctx.gemm(qtype, wd, rows, cols, xd, batch, cols, y, rows)
    ys = []
    for b in range(batch):
        yb = empty_f32(torch_gpu, rows)
        ctx.gemv(qtype, wd, rows, cols, xd[b], yb)
        ys.append(yb)
    ctx.synchronize()
    W, A = _dequant_bound(cpuref, qtype, w, rows, cols)
    tol = 2 * gamma(cols + 4) * (np.abs(xb.astype(np.float64)) @ A.T)
    diff = np.abs(y.view(batch, rows).cpu().numpy() - torch_gpu.stack(ys).cpu().numpy())
    assert np.all(diff <= tol)


def test_stream_read(ctx, torch_gpu):
    """The streaming-read probe takes aligned buffers and is timed under the
    launch profiler; unaligned sizes and pointers are refused."""
    buf = torch_gpu.ones(1 << 20, dtype=torch_gpu.float32, device="cuda")
    ctx.profile(True)
    ctx.stream_read(buf, 4 << 20)
    ctx.stream_read(buf, 64)
    stats = ctx.profile_read()
    ctx.profile(False)
    assert stats["stream read 4194304"][0] == 1 and stats["stream read 64"][0] == 1
    with pytest.raises(l3p.L3PError):
        ctx.stream_read(buf, 100)
    with pytest.raises(l3p.L3PError):
        ctx.stream_read(buf[1:], 64)
