"""Seeded synthetic inputs and a minimal GGUF writer.

Used by tests and by ``bench.py`` to build block-quantized weights and whole
models without any download.  The block byte layouts are GGML's
(llama3pure-c-engine.c:127-195); the value distributions are the benchmark
configurations':

* Q8_0: quants uniform in [-127, 127], fp16 scale |N(0, 0.02)| / 127;
* Q4_0: nibbles uniform in [0, 15], fp16 scale |N(0, 0.02)| / 8;
* Q4_K: every scale and quant byte uniform, d and dmin |N(0, 0.02)| / (15*63);
* Q6_K: ql, qh uniform, int8 sub-scales uniform, d |N(0, 0.02)| / (32*127);
* the other types likewise: every code and sub-scale byte uniform, fp16
  scales |N(0, 0.02)| over the code range (offsets N(0, 0.02)), F16 / BF16
  values N(0, 0.02);
* activations N(0, 1) fp32.

Model weights are drawn N(0, std) in fp32 and block-quantized with the
llama.cpp reference quantizers (round-to-nearest-even fp16 scales).
"""
from __future__ import annotations

import struct

import numpy as np

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, BF16 = 10, 11, 12, 13, 14, 20, 29
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144),
         Q5_K: (256, 176), Q6_K: (256, 210), IQ4_NL: (32, 18)}
# IQ4_NL code book (llama3pure-c-engine.c:204-206)
IQ4_NL_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int8)


def row_bytes(qtype: int, cols: int) -> int:
    e, b = BLOCK[qtype]
    return cols // e * b


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(v.shape + (2,))


def _bf16_bytes(v: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bytes, rounded to nearest even (finite inputs)."""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    h = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.ascontiguousarray(h).view(np.uint8).reshape(v.shape + (2,))


def random_blocks(qtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """uint8 [rows, row_bytes] of random blocks with the configured distribution."""
    rng = np.random.default_rng(seed)
    e, bb = BLOCK[qtype]
    nb = cols // e
    out = np.empty((rows, nb, bb), np.uint8)
    if qtype == Q8_0:
        out[:, :, 0:2] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / 127)
        out[:, :, 2:] = rng.integers(-127, 128, (rows, nb, 32), dtype=np.int8).view(np.uint8)
    elif qtype == Q4_0:
        out[:, :, 0:2] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / 8)
        out[:, :, 2:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
    elif qtype == Q4_K:
        out[:, :, 0:2] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (15 * 63))
        out[:, :, 2:4] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (15 * 63))
        out[:, :, 4:] = rng.integers(0, 256, (rows, nb, 140), dtype=np.uint8)
    elif qtype == Q6_K:
        out[:, :, 0:208] = rng.integers(0, 256, (rows, nb, 208), dtype=np.uint8)
        out[:, :, 208:210] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (32 * 127))
    elif qtype in (Q4_1, Q5_1):
        out[:, :, 0:2] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (8 if qtype == Q4_1 else 16))
        out[:, :, 2:4] = _f16_bytes(rng.normal(0, 0.02, (rows, nb)))
        out[:, :, 4:] = rng.integers(0, 256, (rows, nb, bb - 4), dtype=np.uint8)
    elif qtype == Q5_0:
        out[:, :, 0:2] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / 16)
        out[:, :, 2:] = rng.integers(0, 256, (rows, nb, 20), dtype=np.uint8)
    elif qtype == IQ4_NL:
        out[:, :, 0:2] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / 127)
        out[:, :, 2:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
    elif qtype == Q2_K:
        out[:, :, 0:80] = rng.integers(0, 256, (rows, nb, 80), dtype=np.uint8)
        out[:, :, 80:82] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (3 * 15))
        out[:, :, 82:84] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (3 * 15))
    elif qtype == Q3_K:
        out[:, :, 0:108] = rng.integers(0, 256, (rows, nb, 108), dtype=np.uint8)
        out[:, :, 108:110] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (4 * 32))
    elif qtype == Q5_K:
        out[:, :, 0:2] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (31 * 63))
        out[:, :, 2:4] = _f16_bytes(np.abs(rng.normal(0, 0.02, (rows, nb))) / (31 * 63))
        out[:, :, 4:] = rng.integers(0, 256, (rows, nb, 172), dtype=np.uint8)
    elif qtype == F16:
        out[:, :, :] = _f16_bytes(rng.normal(0, 0.02, (rows, nb)))
    elif qtype == BF16:
        out[:, :, :] = _bf16_bytes(rng.normal(0, 0.02, (rows, nb)).astype(np.float32))
    elif qtype == F32:
        out[:, :, :] = rng.normal(0, 0.02, (rows, nb)).astype(np.float32).view(np.uint8).reshape(rows, nb, 4)
    else:
        raise ValueError(f"no synthetic generator for type {qtype}")
    return out.reshape(rows, nb * bb)


def random_x(n: int, seed: int, batch: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    shape = (n,) if batch is None else (batch, n)
    return rng.standard_normal(shape, dtype=np.float32)


# ---------------------------------------------------------------------------
# weight quantizers (llama.cpp reference semantics, RNE fp16 scales)
# ---------------------------------------------------------------------------

def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """fp32 [rows, cols] -> Q8_0 bytes [rows, cols/32*34]."""
    rows, cols = w.shape
    b = w.reshape(rows, cols // 32, 32).astype(np.float32)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d > 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    t = (b * inv[:, :, None]).astype(np.float64)
    q = np.clip(np.trunc(t + np.copysign(0.5, t)), -127, 127)   # roundf: half away from zero
    out = np.empty((rows, cols // 32, 34), np.uint8)
    out[:, :, 0:2] = _f16_bytes(d)
    out[:, :, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(rows, -1)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """fp32 [rows, cols] -> Q4_0 bytes, llama.cpp quantize_row_q4_0_ref."""
    rows, cols = w.shape
    b = w.reshape(rows, cols // 32, 32).astype(np.float32)
    idx = np.abs(b).argmax(axis=2)
    mx = np.take_along_axis(b, idx[:, :, None], axis=2)[:, :, 0]
    d = (mx / np.float32(-8)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.minimum(15, (b * inv[:, :, None] + np.float32(8.5)).astype(np.int8)).astype(np.uint8)
    out = np.empty((rows, cols // 32, 18), np.uint8)
    out[:, :, 0:2] = _f16_bytes(d)
    out[:, :, 2:] = q[:, :, :16] | (q[:, :, 16:] << 4)
    return out.reshape(rows, -1)


def _round_div(a: np.ndarray, b: np.ndarray, lo: int, hi: int) -> np.ndarray:
    """clip(round(a / b), lo, hi) with 0 where b == 0."""
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(b > 0, np.rint(a / np.where(b > 0, b, 1)), 0)
    return np.clip(r, lo, hi).astype(np.int64)


def quantize_q4_k(w: np.ndarray) -> np.ndarray:
    """fp32 [rows, cols] -> Q4_K bytes [rows, cols/256*144].  A plain min/max
    quantizer (not llama.cpp's iterative search): per 32-element sub-block
    scale (max-min)/15 and offset -min, both stored as 6-bit multiples of the
    fp16 super-block d / dmin; fields packed as get_scale_min_k4 reads them
    (llama3pure-c-engine.c:705-746)."""
    rows, cols = w.shape
    nsb = cols // 256
    b = w.reshape(rows, nsb, 8, 32).astype(np.float32)
    mn = np.minimum(b.min(axis=3), 0)
    scale = (b.max(axis=3) - mn) / np.float32(15)
    off = -mn
    d = (scale.max(axis=2) / np.float32(63)).astype(np.float16)
    dmin = (off.max(axis=2) / np.float32(63)).astype(np.float16)
    dd, dm = d.astype(np.float32), dmin.astype(np.float32)
    sc = _round_div(scale, dd[:, :, None], 0, 63)
    m = _round_div(off, dm[:, :, None], 0, 63)
    d1 = (dd[:, :, None] * sc).astype(np.float32)
    m1 = (dm[:, :, None] * m).astype(np.float32)
    q = _round_div(b + m1[..., None], d1[..., None], 0, 15)
    out = np.empty((rows, nsb, 144), np.uint8)
    out[:, :, 0:2] = np.ascontiguousarray(d).view(np.uint8).reshape(rows, nsb, 2)
    out[:, :, 2:4] = np.ascontiguousarray(dmin).view(np.uint8).reshape(rows, nsb, 2)
    out[:, :, 4:16] = _pack_k4_scales(sc, m)
    qs = q[:, :, 0::2, :] | (q[:, :, 1::2, :] << 4)          # [rows, nsb, 4, 32]
    out[:, :, 16:] = qs.reshape(rows, nsb, 128).astype(np.uint8)
    return out.reshape(rows, -1)


def quantize_q6_k(w: np.ndarray) -> np.ndarray:
    """fp32 [rows, cols] -> Q6_K bytes [rows, cols/256*210]: per 16-element
    group scale max|w|/31 stored as an int8 multiple of the fp16 d, quants
    q = round(w / (d*sc)) in [-32, 31] kept as u = q + 32 in the ql/qh
    layout dequantize_row_q6_K reads (llama3pure-c-engine.c:873-904)."""
    rows, cols = w.shape
    nsb = cols // 256
    b = w.reshape(rows, nsb, 16, 16).astype(np.float32)
    s = np.abs(b).max(axis=3) / np.float32(31)
    d = (s.max(axis=2) / np.float32(127)).astype(np.float16)
    dd = d.astype(np.float32)
    sc = _round_div(s, dd[:, :, None], -128, 127)
    ds = (dd[:, :, None] * sc).astype(np.float32)
    u = (_round_div(b, ds[..., None], -32, 31) + 32).reshape(rows, nsb, 2, 4, 32)   # [.., h, g, l]
    out = np.empty((rows, nsb, 210), np.uint8)
    ql = np.empty((rows, nsb, 2, 64), np.int64)
    ql[..., :32] = (u[:, :, :, 0] & 15) | ((u[:, :, :, 2] & 15) << 4)
    ql[..., 32:] = (u[:, :, :, 1] & 15) | ((u[:, :, :, 3] & 15) << 4)
    qh = (u[:, :, :, 0] >> 4) | ((u[:, :, :, 1] >> 4) << 2) | ((u[:, :, :, 2] >> 4) << 4) | ((u[:, :, :, 3] >> 4) << 6)
    out[:, :, 0:128] = ql.reshape(rows, nsb, 128).astype(np.uint8)
    out[:, :, 128:192] = qh.reshape(rows, nsb, 64).astype(np.uint8)
    out[:, :, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, :, 208:210] = np.ascontiguousarray(d).view(np.uint8).reshape(rows, nsb, 2)
    return out.reshape(rows, -1)


def _h16(v: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 values (RNE) and their bytes."""
    h = v.astype(np.float16)
    return h, np.ascontiguousarray(h).view(np.uint8).reshape(v.shape + (2,))


def _pack_k4_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Eight 6-bit scales and mins [.., 8] -> the 12 bytes get_scale_min_k4
    reads (llama3pure-c-engine.c:705-714)."""
    s = np.empty(sc.shape[:-1] + (12,), np.int64)
    s[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    s[..., 4:8] = (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6)
    s[..., 8:12] = (sc[..., 4:8] & 15) | ((m[..., 4:8] & 15) << 4)
    return s.astype(np.uint8)


def _minmax_32(w: np.ndarray, levels: int):
    """Per 32-block min/max quantization to 0..levels: fp16 d, m, codes."""
    rows, cols = w.shape
    b = w.reshape(rows, cols // 32, 32).astype(np.float32)
    mn, mx = b.min(axis=2), b.max(axis=2)
    d, db = _h16((mx - mn) / np.float32(levels))
    m, mb = _h16(mn)
    q = _round_div(b - m.astype(np.float32)[..., None], d.astype(np.float32)[..., None], 0, levels)
    return db, mb, q


def _qh_bits(q: np.ndarray) -> np.ndarray:
    """Bit 4 of each of the 32 codes of a block -> the 4 qh bytes (bit j = code j)."""
    bits = ((q >> 4) & 1) << np.arange(32, dtype=np.int64)
    v = bits.sum(axis=-1)
    return np.stack([(v >> (8 * k)) & 0xFF for k in range(4)], axis=-1).astype(np.uint8)


def quantize_q4_1(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q4_1 {fp16 d, m; nibbles}: per block d = (max-min)/15, m = min."""
    db, mb, q = _minmax_32(w, 15)
    out = np.empty(q.shape[:2] + (20,), np.uint8)
    out[..., 0:2], out[..., 2:4] = db, mb
    out[..., 4:] = (q[..., :16] | (q[..., 16:] << 4)).astype(np.uint8)
    return out.reshape(w.shape[0], -1)


def quantize_q5_1(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q5_1 {fp16 d, m; qh[4]; nibbles}: per block d = (max-min)/31."""
    db, mb, q = _minmax_32(w, 31)
    out = np.empty(q.shape[:2] + (24,), np.uint8)
    out[..., 0:2], out[..., 2:4] = db, mb
    out[..., 4:8] = _qh_bits(q)
    out[..., 8:] = ((q[..., :16] & 15) | ((q[..., 16:] & 15) << 4)).astype(np.uint8)
    return out.reshape(w.shape[0], -1)


def quantize_q5_0(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q5_0 {fp16 d; qh[4]; nibbles}: d = (signed max)/-16, code
    min(31, trunc(w/d + 16.5)) as in llama.cpp's quantize_row_q5_0_ref."""
    rows, cols = w.shape
    b = w.reshape(rows, cols // 32, 32).astype(np.float32)
    idx = np.abs(b).argmax(axis=2)
    mx = np.take_along_axis(b, idx[:, :, None], axis=2)[:, :, 0]
    d, db = _h16(mx / np.float32(-16))
    dd = d.astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(dd != 0, np.float32(1) / dd, np.float32(0)).astype(np.float32)
    q = np.clip(np.trunc(b * inv[:, :, None] + np.float32(16.5)), 0, 31).astype(np.int64)
    out = np.empty((rows, cols // 32, 22), np.uint8)
    out[..., 0:2] = db
    out[..., 2:6] = _qh_bits(q)
    out[..., 6:] = ((q[..., :16] & 15) | ((q[..., 16:] & 15) << 4)).astype(np.uint8)
    return out.reshape(rows, -1)


def quantize_iq4_nl(w: np.ndarray) -> np.ndarray:
    """fp32 -> IQ4_NL {fp16 d; nibbles}: d = max|w|/127, each value the
    nearest code-book entry."""
    rows, cols = w.shape
    b = w.reshape(rows, cols // 32, 32).astype(np.float32)
    d, db = _h16(np.abs(b).max(axis=2) / np.float32(127))
    dd = d.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = np.where(dd[..., None] > 0, b / np.where(dd > 0, dd, 1)[..., None], 0)
    q = np.abs(t[..., None] - IQ4_NL_VALUES.astype(np.float32)).argmin(axis=-1)
    out = np.empty((rows, cols // 32, 18), np.uint8)
    out[..., 0:2] = db
    out[..., 2:] = (q[..., :16] | (q[..., 16:] << 4)).astype(np.uint8)
    return out.reshape(rows, -1)


def quantize_q2_k(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q2_K {scales[16]; qs[64]; fp16 d, dmin}: per 16-element group
    scale (max-min)/3 and offset -min as 4-bit multiples of d and dmin,
    2-bit codes at the byte and shift dequantize_row_q2_K reads
    (llama3pure-c-engine.c:748-784)."""
    rows, cols = w.shape
    nsb = cols // 256
    b = w.reshape(rows, nsb, 16, 16).astype(np.float32)
    mn = np.minimum(b.min(axis=3), 0)
    scale, off = (b.max(axis=3) - mn) / np.float32(3), -mn
    d, db = _h16(scale.max(axis=2) / np.float32(15))
    dmin, dmb = _h16(off.max(axis=2) / np.float32(15))
    dd, dm = d.astype(np.float32), dmin.astype(np.float32)
    sc = _round_div(scale, dd[..., None], 0, 15)
    m = _round_div(off, dm[..., None], 0, 15)
    u = _round_div(b + (dm[..., None] * m)[..., None], (dd[..., None] * sc)[..., None], 0, 3)
    u = u.reshape(rows, nsb, 2, 4, 2, 16)          # group g = 8*half + 2*j + second
    qs = sum(u[:, :, :, j] << (2 * j) for j in range(4))   # [rows, nsb, half, second, l]
    out = np.empty((rows, nsb, 84), np.uint8)
    out[..., 0:16] = (sc | (m << 4)).astype(np.uint8)
    out[..., 16:80] = qs.reshape(rows, nsb, 64).astype(np.uint8)
    out[..., 80:82], out[..., 82:84] = db, dmb
    return out.reshape(rows, -1)


def quantize_q3_k(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q3_K {hmask[32]; qs[64]; scales[12]; fp16 d}: per 16-element
    group scale max|w|/4 stored as 32 + a 5-bit multiple of d, values in
    [-4, 3] as 2 low bits in qs and a high bit (set for v >= 0) in hmask
    (llama3pure-c-engine.c:786-832)."""
    rows, cols = w.shape
    nsb = cols // 256
    b = w.reshape(rows, nsb, 16, 16).astype(np.float32)
    s = np.abs(b).max(axis=3) / np.float32(4)
    d, db = _h16(s.max(axis=2) / np.float32(31))
    dd = d.astype(np.float32)
    sv = _round_div(s, dd[..., None], 0, 31) + 32                 # 6-bit scale codes
    ds = dd[..., None] * (sv - 32)
    with np.errstate(divide="ignore", invalid="ignore"):
        v = np.where(ds[..., None] > 0, np.rint(b / np.where(ds > 0, ds, 1)[..., None]), 0)
    v = np.clip(v, -4, 3).astype(np.int64)
    q2 = np.where(v >= 0, v, v + 4).reshape(rows, nsb, 2, 4, 2, 16)
    h = (v >= 0).astype(np.int64).reshape(rows, nsb, 2, 4, 2, 16)
    qs = sum(q2[:, :, :, j] << (2 * j) for j in range(4))                       # [.., half, second, l]
    hm = sum(h[:, :, half, j] << (4 * half + j) for half in range(2) for j in range(4))   # [.., second, l]
    sc = np.empty((rows, nsb, 12), np.int64)
    sc[..., 0:8] = (sv[..., 0:8] & 15) | ((sv[..., 8:16] & 15) << 4)
    sc[..., 8:12] = sum(((sv[..., 4 * k:4 * k + 4] >> 4) & 3) << (2 * k) for k in range(4))
    out = np.empty((rows, nsb, 110), np.uint8)
    out[..., 0:32] = hm.reshape(rows, nsb, 32).astype(np.uint8)
    out[..., 32:96] = qs.reshape(rows, nsb, 64).astype(np.uint8)
    out[..., 96:108] = sc.astype(np.uint8)
    out[..., 108:110] = db
    return out.reshape(rows, -1)


def quantize_q5_k(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q5_K {fp16 d, dmin; scales[12]; qh[32]; qs[128]}: the Q4_K
    min/max quantizer with 32 levels, bit 4 of sub-block k's codes in bit k
    of qh (llama3pure-c-engine.c:834-871)."""
    rows, cols = w.shape
    nsb = cols // 256
    b = w.reshape(rows, nsb, 8, 32).astype(np.float32)
    mn = np.minimum(b.min(axis=3), 0)
    scale, off = (b.max(axis=3) - mn) / np.float32(31), -mn
    d, db = _h16(scale.max(axis=2) / np.float32(63))
    dmin, dmb = _h16(off.max(axis=2) / np.float32(63))
    dd, dm = d.astype(np.float32), dmin.astype(np.float32)
    sc = _round_div(scale, dd[..., None], 0, 63)
    m = _round_div(off, dm[..., None], 0, 63)
    q = _round_div(b + (dm[..., None] * m)[..., None], (dd[..., None] * sc)[..., None], 0, 31)
    out = np.empty((rows, nsb, 176), np.uint8)
    out[..., 0:2], out[..., 2:4] = db, dmb
    out[..., 4:16] = _pack_k4_scales(sc, m)
    out[..., 16:48] = sum(((q[:, :, k] >> 4) & 1) << k for k in range(8)).astype(np.uint8)
    out[..., 48:] = ((q[:, :, 0::2] & 15) | ((q[:, :, 1::2] & 15) << 4)).reshape(rows, nsb, 128).astype(np.uint8)
    return out.reshape(rows, -1)


def quantize(w: np.ndarray, qtype: int) -> np.ndarray:
    if qtype == Q8_0:
        return quantize_q8_0(w)
    if qtype == Q4_0:
        return quantize_q4_0(w)
    if qtype == Q4_K:
        return quantize_q4_k(w)
    if qtype == Q6_K:
        return quantize_q6_k(w)
    if qtype == F32:
        return np.ascontiguousarray(w, np.float32).view(np.uint8).reshape(w.shape[0], -1)
    if qtype == F16:
        return _f16_bytes(np.asarray(w, np.float32)).reshape(w.shape[0], -1)
    if qtype == BF16:
        return _bf16_bytes(np.asarray(w, np.float32)).reshape(w.shape[0], -1)
    other = {Q4_1: quantize_q4_1, Q5_0: quantize_q5_0, Q5_1: quantize_q5_1, IQ4_NL: quantize_iq4_nl,
             Q2_K: quantize_q2_k, Q3_K: quantize_q3_k, Q5_K: quantize_q5_k}
    if qtype in other:
        return other[qtype](w)
    raise ValueError(f"no weight quantizer for type {qtype}")


# ---------------------------------------------------------------------------
# GGUF writer (v3, little endian; layout per llama3pure-c-engine.c:2500-2688)
# ---------------------------------------------------------------------------

_GT_U32, _GT_I32, _GT_F32, _GT_STR, _GT_ARR = 4, 5, 6, 8, 9


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, val) -> bytes:
    k = _s(key.encode())
    if isinstance(val, str):
        return k + struct.pack("<I", _GT_STR) + _s(val.encode())
    if isinstance(val, float):
        return k + struct.pack("<If", _GT_F32, val)
    if isinstance(val, int):
        return k + struct.pack("<II", _GT_U32, val)
    if isinstance(val, list):   # list of str
        body = b"".join(_s(v.encode()) for v in val)
        return k + struct.pack("<IIQ", _GT_ARR, _GT_STR, len(val)) + body
    raise TypeError(type(val))


def _gguf_header(meta: dict, specs: list, alignment: int):
    """Header bytes and the data offset of every tensor (relative to the data start)."""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(specs), len(meta)))
    for k, v in meta.items():
        head += _kv(k, v)
    off = 0
    offsets = []
    for name, qtype, ne, nbytes in specs:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        head += _s(name.encode()) + struct.pack("<I", len(ne))
        for n in ne:
            head += struct.pack("<Q", n)
        head += struct.pack("<IQ", qtype, off)
        off += nbytes
    head += bytes((-len(head)) % alignment)
    return bytes(head), offsets, off


def build_gguf(meta: dict, specs: list, fill, alignment: int = 32) -> np.ndarray:
    """GGUF v3 image in one preallocated uint8 array.  specs: (name, qtype, ne, nbytes);
    fill(i, view) writes tensor i's raw bytes into view (called in spec order)."""
    head, offsets, data = _gguf_header(meta, specs, alignment)
    out = np.zeros(len(head) + data, np.uint8)
    out[:len(head)] = np.frombuffer(head, np.uint8)
    for i, ((name, qtype, ne, nbytes), o) in enumerate(zip(specs, offsets)):
        fill(i, out[len(head) + o: len(head) + o + nbytes])
    return out


def write_gguf(meta: dict, tensors: list, alignment: int = 32) -> bytes:
    """tensors: list of (name, qtype, ne (cols, rows) or (n,), raw uint8 bytes)."""
    specs = [(n, q, ne, len(raw)) for n, q, ne, raw in tensors]

    def fill(i, view):
        view[:] = np.frombuffer(bytes(tensors[i][3]), np.uint8)

    return build_gguf(meta, specs, fill, alignment).tobytes()


def synthetic_model(arch: str = "llama", dim: int = 256, hidden: int = 512, n_layers: int = 2,
                    n_heads: int = 8, n_kv: int = 2, head_dim: int | None = None, vocab: int = 512,
                    ctx: int = 256, qtype: int = Q8_0, std: float = 0.02, seed: int = 0,
                    rope_theta: float = 500000.0, eps: float = 1e-5, tied: bool = False,
                    softcap: float = 0.0, swa_window: int = 0, rope_theta_swa: float = 10000.0,
                    norm_jitter: float = 0.0, qtypes: dict | None = None, make_mat=None,
                    mats: dict | None = None):
    """A random-init model in GGUF form.  arch 'llama' (Llama-3 layout) or
    'gemma3' (Gemma layout: QK-norm, post norms, NEOX RoPE, GeGLU).
    qtypes overrides the type per tensor-name suffix (e.g. {"ffn_down": Q4_0}).
    make_mat(qtype, rows, cols, std, view), when given, writes the quantized
    bytes of each matrix into view (e.g. generated on a GPU for multi-GB
    models) and the image is returned as a uint8 array instead of bytes.
    mats maps tensor names to fp32 [rows, cols] matrices that replace the
    random ones (quantized to the tensor's type)."""
    rng = np.random.default_rng(seed)
    hd = head_dim or dim // n_heads
    qd, kvd = n_heads * hd, n_kv * hd
    pre = "gemma3" if arch.startswith("gemma") else "llama"
    meta = {
        "general.architecture": arch,
        f"{pre}.embedding_length": dim,
        f"{pre}.feed_forward_length": hidden,
        f"{pre}.block_count": n_layers,
        f"{pre}.attention.head_count": n_heads,
        f"{pre}.attention.head_count_kv": n_kv,
        f"{pre}.vocab_size": vocab,
        f"{pre}.context_length": ctx,
        f"{pre}.rope.freq_base": float(rope_theta),
        f"{pre}.attention.key_length": hd,
        f"{pre}.attention.layer_norm_rms_epsilon": float(eps),
    }
    if pre == "gemma3":
        meta[f"{pre}.final_logit_softcapping"] = float(softcap)
        meta[f"{pre}.attention.sliding_window"] = swa_window
        meta[f"{pre}.rope.freq_base_swa"] = float(rope_theta_swa)
    meta["tokenizer.ggml.tokens"] = [f"<t{i}>" for i in range(vocab)]
    meta["tokenizer.ggml.bos_token_id"] = 1
    meta["tokenizer.ggml.eos_token_id"] = 2

    def qtype_of(name):
        t = qtype
        for k, v in (qtypes or {}).items():
            if k in name:
                t = v
        return t

    # (name, kind, rows, cols): kind "mat" (quantized, ne = (cols, rows)) or "norm" (F32, ne = (n,))
    layout = [("token_embd.weight", "mat", vocab, dim)]
    for l in range(n_layers):
        p = f"blk.{l}."
        layout += [(p + "attn_norm.weight", "norm", dim, 1),
                   (p + "attn_q.weight", "mat", qd, dim),
                   (p + "attn_k.weight", "mat", kvd, dim),
                   (p + "attn_v.weight", "mat", kvd, dim),
                   (p + "attn_output.weight", "mat", dim, qd),
                   (p + "ffn_norm.weight", "norm", dim, 1),
                   (p + "ffn_gate.weight", "mat", hidden, dim),
                   (p + "ffn_down.weight", "mat", dim, hidden),
                   (p + "ffn_up.weight", "mat", hidden, dim)]
        if pre == "gemma3":
            layout += [(p + "attn_q_norm.weight", "norm", hd, 1),
                       (p + "attn_k_norm.weight", "norm", hd, 1),
                       (p + "post_attention_norm.weight", "norm", dim, 1),
                       (p + "post_ffw_norm.weight", "norm", dim, 1)]
    layout.append(("output_norm.weight", "norm", dim, 1))
    if not tied:
        layout.append(("output.weight", "mat", vocab, dim))

    specs = []
    for name, kind, rows, cols in layout:
        if kind == "mat":
            t = qtype_of(name)
            specs.append((name, t, (cols, rows), rows * row_bytes(t, cols)))
        else:
            specs.append((name, F32, (rows,), 4 * rows))

    def fill(i, view):
        name, kind, rows, cols = layout[i]
        if kind == "norm":
            v = np.ones(rows, np.float32)
            if norm_jitter:
                v += rng.normal(0, norm_jitter, rows).astype(np.float32)
            view[:] = v.view(np.uint8)
        elif make_mat is not None:
            make_mat(specs[i][1], rows, cols, std, view)
        else:
            w = rng.normal(0, std, (rows, cols)).astype(np.float32)
            if mats and name in mats:
                w = np.ascontiguousarray(mats[name], np.float32).reshape(rows, cols)
            view[:] = quantize(w, specs[i][1]).ravel()

    out = build_gguf(meta, specs, fill)
    return out if make_mat is not None else out.tobytes()


def gpu_q8_0_maker(ctx, torch, seed: int):
    """make_mat for synthetic_model that draws each matrix N(0, std) on the GPU
    (torch's generator, seeded) and quantizes it to Q8_0 blocks with the
    library's quantizer (l3p_quantize_q8_0), for multi-GB models that numpy
    would take minutes to quantize.  ctx is an llama3pure_amd.Context."""
    st = torch.cuda.ExternalStream(ctx.stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)

    def make(qtype, rows, cols, std, view):
        assert qtype == Q8_0, "the GPU maker writes Q8_0 blocks only"
        rb = cols // 32 * 34
        step = max(1, (1 << 26) // cols)
        with torch.cuda.stream(st):
            for r0 in range(0, rows, step):
                n = min(step, rows - r0)
                w = torch.randn(n * cols, device="cuda", generator=gen) * std
                q = torch.empty(n * rb, dtype=torch.uint8, device="cuda")
                ctx.quantize_q8_0(w, n * cols, q)
                view[r0 * rb:(r0 + n) * rb] = q.cpu().numpy()
        return view

    return make
