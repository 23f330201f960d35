"""Pins for the oracle's primitives (oracle/cpuref.c), CPU only.

Each primitive is checked against (a) what the mathematics fixes, computed
independently here (IEEE binary16, exact rationals, float64 bounds), and
(b) the reference engine itself where oracle/_ref was built.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle
from block_math import codes_32
from llama3pure_amd import synth

ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def rn32(fr: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32 (ties to even)."""
    f = np.float32(float(fr))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - fr)
        if best is None or d < best[0] or (d == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (d, c)
    return np.float32(best[1])


# --------------------------------------------------------------------------- fp16
def test_fp16_to_fp32_exhaustive_ieee(cpuref):
    """c:547-582 is IEEE binary16 -> binary32 for every non-NaN code."""
    got = cpuref.fp16_to_fp32(ALL16)
    want = ALL16.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaN codes keep sign and payload, exponent all ones (no quiet bit forced)
    h = ALL16[nan].astype(np.uint32)
    exp_bits = ((h & 0x8000) << 16) | 0x7F800000 | ((h & 0x3FF) << 13)
    assert np.array_equal(got[nan].view(np.uint32), exp_bits)


def test_fp16_table_matches_reference(cpuref, refc):
    sample = ALL16[::7]
    assert np.array_equal(cpuref.fp16_to_fp32(sample).view(np.uint32), refc.fp16_to_fp32(sample).view(np.uint32))


def _rtz16(f: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 rounding toward zero, from numpy's RNE conversion."""
    with np.errstate(over="ignore"):
        h = f.astype(np.float16)
    hb = h.view(np.uint16).copy()
    back = h.astype(np.float32)
    over = np.abs(back) > np.abs(f)     # RNE rounded away from zero: step one code toward zero
    hb[over] -= 1
    return hb


def test_fp32_to_fp16_truncates_toward_zero(cpuref):
    """c:585-599 truncates: every finite value below 65536 maps to its
    round-toward-zero binary16; |x| >= 65536 and NaN map to signed inf."""
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    got = cpuref.fp32_to_fp16(f)
    small = np.abs(f) < 65536
    assert np.array_equal(got[small], _rtz16(f[small]))
    big = ~small
    assert np.all((got[big] & 0x7FFF) == 0x7C00)
    assert np.array_equal(got[big] >> 15, (f[big] < 0).astype(np.uint16))
    # edge classes
    edges = np.array([0.0, -0.0, 2**-24, 2**-25, 2**-24 * 1.5, 2**-14, 2**-14 * (1 - 2**-11), 65504, 65519.99,
                      65520, 1.0 + 2**-11, 1.0 + 2**-10 - 2**-20, -3.0e-8], np.float32)
    got = cpuref.fp32_to_fp16(edges)
    want = np.where(np.abs(edges) < 65536, _rtz16(edges), 0x7C00 | ((edges < 0) << 15).astype(np.uint16))
    assert np.array_equal(got, want.astype(np.uint16))
    nan_inf = cpuref.fp32_to_fp16(np.array([np.nan, np.inf, -np.inf], np.float32))
    assert list(nan_inf) == [0x7C00, 0x7C00, 0xFC00]


def test_fp32_to_fp16_matches_reference(cpuref, refc):
    rng = np.random.default_rng(1)
    f = rng.standard_normal(50000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 50000)
    f = f.astype(np.float32)
    assert np.array_equal(cpuref.fp32_to_fp16(f), refc.fp32_to_fp16(f))


# --------------------------------------------------------------------------- dequant
def _fp16(b):
    return Fraction(float(np.frombuffer(bytes(b), np.float16)[0]))


def _neg16(b):
    return bool(b[1] & 0x80)


def _mul(av, aneg, bv, bneg):
    """Exact product with the IEEE sign of a zero result: (value, is_negative)."""
    return av * bv, aneg != bneg


def _exact_dequant_block(qtype, blk):
    """Exact rational values of one block, from the GGML format definition,
    as (value, sign) pairs; the sign only matters for zeros (IEEE: the sign of
    a product is the XOR of the operand signs, x - x is +0)."""
    blk = [int(v) for v in blk]
    s8 = lambda v: v - 256 if v > 127 else v
    if qtype == oracle.Q8_0:
        d, dn = _fp16(blk[0:2]), _neg16(blk[0:2])
        return [_mul(Fraction(s8(v)), s8(v) < 0, d, dn) for v in blk[2:34]]
    if qtype == oracle.Q4_0:
        d, dn = _fp16(blk[0:2]), _neg16(blk[0:2])
        q = [(blk[2 + j] & 15) - 8 for j in range(16)] + [(blk[2 + j] >> 4) - 8 for j in range(16)]
        return [_mul(Fraction(v), v < 0, d, dn) for v in q]
    if qtype == oracle.Q4_K:
        d, dn = _fp16(blk[0:2]), _neg16(blk[0:2])
        dmin, mn = _fp16(blk[2:4]), _neg16(blk[2:4])
        s = blk[4:16]
        out = []
        for j in range(8):
            if j < 4:
                sc, m = s[j] & 63, s[j + 4] & 63
            else:
                sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
                m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
            q = blk[16 + 32 * (j // 2): 16 + 32 * (j // 2) + 32]
            for n in [(v >> 4) if j % 2 else (v & 15) for v in q]:
                a, an = _mul(*_mul(d, dn, Fraction(sc), False), Fraction(n), False)
                b, bn = _mul(dmin, mn, Fraction(m), False)
                v = a - b
                out.append((v, v == 0 and a == 0 and b == 0 and an and not bn))
        return out
    if qtype == oracle.Q6_K:
        d, dn = _fp16(blk[208:210]), _neg16(blk[208:210])
        out = [None] * 256
        for half in range(2):
            ql, qh = blk[64 * half: 64 * half + 64], blk[128 + 32 * half: 128 + 32 * half + 32]
            sc = [s8(v) for v in blk[192 + 8 * half: 200 + 8 * half]]
            for l in range(32):
                q = [(ql[l] & 15) | (((qh[l] >> 0) & 3) << 4), (ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4),
                     (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4), (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)]
                for g in range(4):
                    c = sc[l // 16 + 2 * g]
                    ds = _mul(d, dn, Fraction(c), c < 0)
                    out[128 * half + 32 * g + l] = _mul(*ds, Fraction(q[g] - 32), q[g] < 32)
        return out
    if qtype in (oracle.Q4_1, oracle.Q5_1):
        # y = q*d + m: q*d is exact, the sum rounds once
        d, dn = _fp16(blk[0:2]), _neg16(blk[0:2])
        m, mn = _fp16(blk[2:4]), _neg16(blk[2:4])
        if qtype == oracle.Q4_1:
            q = [blk[4 + j] & 15 for j in range(16)] + [blk[4 + j] >> 4 for j in range(16)]
        else:
            qh = blk[4] | (blk[5] << 8) | (blk[6] << 16) | (blk[7] << 24)
            q = [(blk[8 + j] & 15) | (((qh >> j) & 1) << 4) for j in range(16)] + \
                [(blk[8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4) for j in range(16)]
        return [_add(*_mul(Fraction(v), False, d, dn), m, mn) for v in q]
    if qtype == oracle.Q5_0:
        d, dn = _fp16(blk[0:2]), _neg16(blk[0:2])
        qh = blk[2] | (blk[3] << 8) | (blk[4] << 16) | (blk[5] << 24)
        q = [(blk[6 + j] & 15) | (((qh >> j) & 1) << 4) for j in range(16)] + \
            [(blk[6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4) for j in range(16)]
        return [_mul(Fraction(v - 16), v < 16, d, dn) for v in q]
    if qtype == oracle.IQ4_NL:
        d, dn = _fp16(blk[0:2]), _neg16(blk[0:2])
        q = [synth.IQ4_NL_VALUES[blk[2 + j] & 15] for j in range(16)] + \
            [synth.IQ4_NL_VALUES[blk[2 + j] >> 4] for j in range(16)]
        return [_mul(d, dn, Fraction(int(v)), v < 0) for v in q]
    if qtype == oracle.Q2_K:
        # 16 groups of 16: group g = 8*half + 2*j + second, 2-bit codes of
        # qs[32*half + 16*second + l] at bit 2*j; y = (d*(s&15))*u - dmin*(s>>4)
        d, dn = _fp16(blk[80:82]), _neg16(blk[80:82])
        dmin, mn = _fp16(blk[82:84]), _neg16(blk[82:84])
        out = []
        for g in range(16):
            half, j, second = g // 8, (g // 2) % 4, g % 2
            sc = blk[g]
            for l in range(16):
                u = (blk[16 + 32 * half + 16 * second + l] >> (2 * j)) & 3
                a, an = _mul(*_mul(d, dn, Fraction(sc & 15), False), Fraction(u), False)
                b, bn = _mul(dmin, mn, Fraction(sc >> 4), False)
                out.append(_sub(a, an, b, bn))
        return out
    if qtype == oracle.Q3_K:
        # 16 groups as Q2_K, value u - 4 unless bit 4*half + j of
        # hmask[16*second + l] is set, scale d*(s_g - 32) with s_g the 6-bit
        # field: low 4 bits from byte g (g < 8) or the high nibble of byte
        # g - 8, high 2 bits from byte 8 + g%4 at bit 2*(g/4)
        d, dn = _fp16(blk[108:110]), _neg16(blk[108:110])
        sb = blk[96:108]
        out = []
        for g in range(16):
            half, j, second = g // 8, (g // 2) % 4, g % 2
            lo = (sb[g] & 15) if g < 8 else (sb[g - 8] >> 4)
            sg = (lo | (((sb[8 + g % 4] >> (2 * (g // 4))) & 3) << 4)) - 32
            ds = _mul(d, dn, Fraction(sg), sg < 0)
            for l in range(16):
                u = (blk[32 + 32 * half + 16 * second + l] >> (2 * j)) & 3
                h = (blk[16 * second + l] >> (4 * half + j)) & 1
                v = u - (0 if h else 4)
                out.append(_mul(*ds, Fraction(v), v < 0))
        return out
    if qtype == oracle.Q5_K:
        d, dn = _fp16(blk[0:2]), _neg16(blk[0:2])
        dmin, mn = _fp16(blk[2:4]), _neg16(blk[2:4])
        s = blk[4:16]
        out = []
        for k in range(8):
            if k < 4:
                sc, m = s[k] & 63, s[k + 4] & 63
            else:
                sc = (s[k + 4] & 0xF) | ((s[k - 4] >> 6) << 4)
                m = (s[k + 4] >> 4) | ((s[k] >> 6) << 4)
            for l in range(32):
                byte = blk[48 + 32 * (k // 2) + l]
                q = ((byte >> 4) if k % 2 else (byte & 15)) + 16 * ((blk[16 + l] >> k) & 1)
                a, an = _mul(*_mul(d, dn, Fraction(sc), False), Fraction(q), False)
                b, bn = _mul(dmin, mn, Fraction(m), False)
                out.append(_sub(a, an, b, bn))
        return out
    raise ValueError(qtype)


def _add(a, an, b, bn):
    """Exact a + b with the IEEE sign of a zero sum (-0 only for -0 + -0)."""
    v = a + b
    return v, v == 0 and a == 0 and b == 0 and an and bn


def _sub(a, an, b, bn):
    """Exact a - b with the IEEE sign of a zero result (-0 only for -0 - +0)."""
    v = a - b
    return v, v == 0 and a == 0 and b == 0 and an and not bn


def _to_f32(vs):
    return np.array([(np.float32(-0.0) if neg else np.float32(0.0)) if v == 0 else rn32(v) for v, neg in vs],
                    np.float32)


@pytest.mark.parametrize("qtype", [oracle.Q8_0, oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.IQ4_NL,
                                   oracle.Q2_K, oracle.Q3_K, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K])
def test_dequant_closed_form(cpuref, qtype):
    """Every dequantized value is the float32 rounding of the exact rational
    the format defines (only the offset additions of Q4_1 / Q5_1 and the
    min subtractions of Q2_K / Q4_K / Q5_K round)."""
    e, bb = oracle.BLOCK[qtype]
    rows = synth.random_blocks(qtype, 1, e * 6, seed=qtype)
    got = cpuref.dequant(qtype, rows[0], e * 6)
    want = np.concatenate([_to_f32(_exact_dequant_block(qtype, rows[0][b * bb:(b + 1) * bb])) for b in range(6)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", [oracle.Q8_0, oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.Q2_K,
                                   oracle.Q3_K, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K, oracle.IQ4_NL, oracle.F16,
                                   oracle.BF16])
def test_dequant_matches_reference(cpuref, refc, qtype):
    e, bb = oracle.BLOCK[qtype]
    n = max(e, 32) * 16
    raw = np.random.default_rng(qtype).integers(0, 256, n // e * bb, dtype=np.uint8)
    if qtype in (oracle.F16, oracle.BF16):
        pass
    got = cpuref.dequant(qtype, raw, n)
    want = refc.dequant(qtype, raw, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------------------- quantizer
def _quantize_closed_form(x):
    """quantize_row_q8_0 (c:1508-1528) from IEEE float32 ops done by numpy."""
    out = []
    for b in range(x.size // 32):
        xb = x[32 * b: 32 * b + 32]
        amax = np.float32(np.max(np.abs(xb))) if xb.size else np.float32(0)
        d = np.float32(amax / np.float32(127.0))
        idv = np.float32(np.float32(127.0) / amax) if d > 0 else np.float32(0)
        v = (xb * idv).astype(np.float32).astype(np.float64)
        q = np.clip(np.trunc(v + np.copysign(0.5, v)), -128, 127).astype(np.int8)   # roundf
        h = _rtz16(np.array([d], np.float32))[0]
        out.append(np.concatenate([np.frombuffer(np.uint16(h).tobytes(), np.uint8), q.view(np.uint8)]))
    return np.concatenate(out)


def test_quantize_q8_0_closed_form(cpuref):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(32 * 64).astype(np.float32) * np.float32(3.0)
    x[:32] = 0.0                                # amax == 0 -> d = 0, q = 0
    x[32:64] = np.arange(32, dtype=np.float32) - 15.5   # ties at .5 after scaling by 127/16.5? (covered below)
    x[64:96] = np.float32(1e-30)                # subnormal scale region
    # exact ties: amax = 127 gives id = 1, so x = k + 0.5 rounds away from zero
    x[96:128] = np.array([127.0] + [k + 0.5 for k in range(-15, 16)], np.float32)
    got = cpuref.quantize_q8_0(x)
    assert np.array_equal(got, _quantize_closed_form(x))
    q = got[96 * 34 // 32 + 2: 96 * 34 // 32 + 34].view(np.int8)
    assert q[1] == -15 and q[16] == 1 and q[-1] == 16   # -14.5 -> -15, 0.5 -> 1, 15.5 -> 16


def test_quantize_q8_0_matches_reference(cpuref, refc):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(32 * 500) * np.float32(10.0) ** rng.integers(-6, 4, 32 * 500)).astype(np.float32)
    assert np.array_equal(cpuref.quantize_q8_0(x), refc.quantize_q8_0(x))


# --------------------------------------------------------------------------- matmul
def gamma(n):
    u = 2.0 ** -24
    return n * u / (1 - n * u)


def _dequant_rows_f64(cpuref, qtype, w, rows, cols):
    return np.stack([cpuref.dequant(qtype, w[r], cols) for r in range(rows)]).astype(np.float64)


@pytest.mark.parametrize("qtype,rows,cols", [(oracle.Q8_0, 37, 512), (oracle.Q2_K, 11, 768), (oracle.Q3_K, 9, 512),
                                             (oracle.Q4_K, 19, 1024), (oracle.Q5_K, 7, 512), (oracle.Q6_K, 13, 512),
                                             (oracle.F16, 5, 320), (oracle.BF16, 6, 256), (oracle.F32, 7, 96)])
def test_matmul_float_bound(cpuref, qtype, rows, cols):
    """Float-input types: |y - y64| <= gamma_K * sum|w x| (any fp32 order)."""
    w = synth.random_blocks(qtype, rows, cols, seed=11)
    x = synth.random_x(cols, seed=12)
    y = cpuref.matmul(qtype, w, rows, cols, x)
    W = _dequant_rows_f64(cpuref, qtype, w, rows, cols)
    y64 = W @ x.astype(np.float64)
    bound = gamma(cols) * (np.abs(W) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - y64) <= bound)
    # a dropped term would exceed the bound for at least one row
    y_bad = (W[:, 1:] @ x[1:].astype(np.float64))
    assert np.any(np.abs(y_bad - y64) > bound)


@pytest.mark.parametrize("qtype", [oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.IQ4_NL])
def test_matmul_q8_activation_integer_path(cpuref, qtype):
    """Q4_0, Q4_1, Q5_0, Q5_1, IQ4_NL: x is quantized to Q8_0 and every block
    contributes dw*dx*isum (+ mw*dx*xsum for the types with a min), isum and
    xsum exact integers: the sum is within gamma of the float64 sum of those
    terms, and dropping a block's min term breaks the bound."""
    rows, cols = 23, 512
    e, bb = oracle.BLOCK[qtype]
    w = synth.random_blocks(qtype, rows, cols, seed=13 + qtype)
    x = synth.random_x(cols, seed=14)
    y = cpuref.matmul(qtype, w, rows, cols, x)
    xq = cpuref.quantize_q8_0(x).reshape(-1, 34)
    dx = xq[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    qx = xq[:, 2:].view(np.int8).astype(np.int64)
    wb = w.reshape(rows, -1, bb)
    dw = wb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    code, mo = codes_32(qtype, wb)
    terms = dw * dx[None] * (code * qx[None]).sum(axis=2)
    if mo is not None:
        mw = wb[:, :, mo:mo + 2].copy().view(np.float16).astype(np.float64)[:, :, 0]
        mterms = mw * dx[None] * qx.sum(axis=1)[None]
        assert np.any(np.abs(y - terms.sum(axis=1)) > gamma(2 * cols // 32 + 2) * np.abs(terms).sum(axis=1))
        terms = terms + mterms
    y64 = terms.sum(axis=1)
    assert np.all(np.abs(y - y64) <= gamma(2 * cols // 32 + 2) * np.abs(terms).sum(axis=1))


@pytest.mark.parametrize("qtype,cols", [(oracle.Q8_0, 256), (oracle.Q4_0, 256), (oracle.Q4_1, 256), (oracle.Q5_0, 288),
                                        (oracle.Q5_1, 256), (oracle.IQ4_NL, 224), (oracle.Q2_K, 512),
                                        (oracle.Q3_K, 768), (oracle.Q4_K, 512), (oracle.Q5_K, 512),
                                        (oracle.Q6_K, 512), (oracle.F16, 192), (oracle.BF16, 160), (oracle.F32, 128)])
def test_matmul_matches_reference(cpuref, refc, qtype, cols):
    rows = 21   # not a multiple of 4: exercises the reference's tail rows
    w = synth.random_blocks(qtype, rows, cols, seed=3)
    x = synth.random_x(cols, seed=4)
    assert np.array_equal(cpuref.matmul(qtype, w, rows, cols, x).view(np.uint32),
                          refc.matmul(qtype, w, rows, cols, x).view(np.uint32))
    xb = synth.random_x(cols, seed=5, batch=5)
    assert np.array_equal(cpuref.matmul_batch(qtype, w, rows, cols, xb).view(np.uint32),
                          refc.matmul_batch(qtype, w, rows, cols, xb).view(np.uint32))


# --------------------------------------------------------------------------- elementwise
def test_fast_math_matches_reference_and_bounds(cpuref, refc):
    xs = np.linspace(-12, 12, 2001).astype(np.float32)
    for v in xs:
        assert np.float32(cpuref.fast_expf(float(v))).view(np.uint32) == np.float32(refc.lib.ref_fast_expf(float(v))).view(np.uint32)
        assert np.float32(cpuref.fast_tanhf(float(v))).view(np.uint32) == np.float32(refc.lib.ref_fast_tanhf(float(v))).view(np.uint32)
    # Pade approximants are within a few 1e-4 relative of the true functions near 0
    for v in (-2.0, -0.5, 0.0, 0.5, 2.0):
        assert abs(cpuref.fast_expf(v) - np.exp(v)) < 2e-3 * np.exp(v)
        assert abs(cpuref.fast_tanhf(v) - np.tanh(v)) < 1e-4


def test_rmsnorm_softmax(cpuref, refc):
    rng = np.random.default_rng(9)
    x = rng.standard_normal(4096).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    o = cpuref.rmsnorm(x, w, 1e-5)
    assert np.array_equal(o.view(np.uint32), refc.rmsnorm(x, w, 1e-5).view(np.uint32))
    x64 = x.astype(np.float64)
    o64 = w * (x64 / np.sqrt(np.mean(x64 * x64) + 1e-5))
    assert np.allclose(o, o64, rtol=1e-5, atol=1e-6)
    s = rng.standard_normal(777).astype(np.float32) * 4
    p = cpuref.softmax(s)
    assert np.array_equal(p.view(np.uint32), refc.softmax(s).view(np.uint32))
    e = np.exp(s.astype(np.float64) - s.max())
    assert np.allclose(p, e / e.sum(), rtol=1e-5, atol=1e-9)


# --------------------------------------------------------------------------- sampler
def test_xorshift_known_answers(cpuref):
    """xorshift64* (c:4266-4276) with multiplier 0x2545F4914F6CDD1D."""
    def step(s):
        s ^= s >> 12
        s ^= (s << 25) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 27
        return s, ((s * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) >> 32
    s, want = 42, []
    for _ in range(8):
        s, u = step(s)
        want.append(u)
    assert cpuref.rng_u32(42, 8) == want


def test_sampler_limits(cpuref):
    rng = np.random.default_rng(2)
    lg = rng.standard_normal(5000).astype(np.float32)
    am = int(np.argmax(lg))
    assert cpuref.sample(lg, 0.0, 40, 0.9, 7)[0] == am
    for seed in range(20):
        assert cpuref.sample(lg, 0.9, 1, 0.9, seed + 1)[0] == am          # k = 1
        assert cpuref.sample(lg, 0.9, 40, 1e-9, seed + 1)[0] == am        # top-p keeps only the best
    # empirical distribution over many draws follows softmax(top-k / T)
    lg2 = np.array([2.0, 1.0, 0.5, 0.0, -1.0] + [-50.0] * 100, np.float32)
    counts = np.zeros(lg2.size)
    st = 123
    for _ in range(20000):
        t, st = cpuref.sample(lg2, 1.0, 5, 1.0, st)
        counts[t] += 1
    p = np.exp(lg2[:5] - 2.0)
    p /= p.sum()
    assert np.allclose(counts[:5] / counts.sum(), p, atol=0.015)


@pytest.mark.parametrize("cap", [0.0, 50.0, 5.0])
def test_attend_head_softcap_closed_form(cpuref, cap):
    """One head's attention with the score cap, a load option the reference
    does not have (Gemma-2's attention logit soft-capping): weights
    softmax(cap * tanh(s / cap)) (cap 0: softmax(s)) and output sum w_t V_t,
    with s the dot of the dequantized Q8_0 q and K rows, all in float64
    here.  Scores reach +-150, so a cap of 50 or 5 moves every weight."""
    rng = np.random.default_rng(21)
    hs, n = 128, 40
    q8 = cpuref.quantize_q8_0(rng.normal(0, 6, hs).astype(np.float32))
    kc = cpuref.quantize_q8_0(rng.normal(0, 1.2, (n, hs)).astype(np.float32).ravel())
    vc = cpuref.quantize_q8_0(rng.normal(0, 1, (n, hs)).astype(np.float32).ravel())
    dq = cpuref.dequant(oracle.Q8_0, q8, hs).astype(np.float64)
    dk = cpuref.dequant(oracle.Q8_0, kc, n * hs).astype(np.float64).reshape(n, hs)
    dv = cpuref.dequant(oracle.Q8_0, vc, n * hs).astype(np.float64).reshape(n, hs)
    s = dk @ dq
    assert np.abs(s).max() > 60
    z = cap * np.tanh(s / cap) if cap > 0 else s
    w = np.exp(z - z.max())
    w /= w.sum()
    att, out = cpuref.attend_head(q8, kc, vc, n, hs, cap)
    assert np.allclose(att, w, rtol=1e-4, atol=1e-7), np.abs(att - w).max()
    assert np.allclose(out, w @ dv, rtol=0, atol=1e-4 * np.abs(w @ dv).max())
    if cap > 0:   # the cap changes the weights: the check above would catch a dropped cap
        raw = np.exp(s - s.max())
        raw /= raw.sum()
        assert np.abs(raw - w).max() > 0.05
