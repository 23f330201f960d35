"""Field extraction of GGML block types in numpy (layouts of
llama3pure-c-engine.c:127-201), shared by the oracle and GPU parity tests:
integer codes of the Q8_0-activation types and the per-element magnitudes
that bound the fp32 rounding of the factored K-quant dots."""
import numpy as np

import oracle
from llama3pure_amd import synth


def f16(a):
    """uint8 [..., 2] fp16 bytes -> float64 values."""
    return np.ascontiguousarray(a).view(np.float16).astype(np.float64)[..., 0]


def codes_32(qtype, wb):
    """Integer codes [rows, blocks, 32] of a 32-element block type (wb =
    [rows, blocks, block_bytes]) and the byte offset of its fp16 min (None
    for the types without one)."""
    if qtype in (oracle.Q4_0, oracle.IQ4_NL):
        nib = np.concatenate([(wb[:, :, 2:] & 15), (wb[:, :, 2:] >> 4)], axis=2).astype(np.int64)
        return (nib - 8 if qtype == oracle.Q4_0 else synth.IQ4_NL_VALUES.astype(np.int64)[nib]), None
    if qtype == oracle.Q4_1:
        return np.concatenate([(wb[:, :, 4:] & 15), (wb[:, :, 4:] >> 4)], axis=2).astype(np.int64), 2
    qo = 6 if qtype == oracle.Q5_0 else 8
    qh = wb[:, :, qo - 4:qo].astype(np.int64)
    qh = qh[..., 0] | (qh[..., 1] << 8) | (qh[..., 2] << 16) | (qh[..., 3] << 24)
    nib = np.concatenate([(wb[:, :, qo:] & 15), (wb[:, :, qo:] >> 4)], axis=2).astype(np.int64)
    code = nib | (((qh[..., None] >> np.arange(32)) & 1) << 4)
    return (code - 16, None) if qtype == oracle.Q5_0 else (code, 2)


def q8_block_terms(cpuref, qtype, w, rows, cols, x):
    """Per-block float64 terms dw*dx*isum (+ mw*dx*xsum) of the types whose
    reference dot takes the activation as Q8_0 (vec_dot_*_q8_0)."""
    e, bb = oracle.BLOCK[qtype]
    xq = cpuref.quantize_q8_0(x).reshape(-1, 34)
    dx = f16(xq[:, 0:2])
    qx = xq[:, 2:].view(np.int8).astype(np.int64)
    wb = w.reshape(rows, -1, bb)
    code, mo = codes_32(qtype, wb)
    terms = f16(wb[:, :, 0:2]) * dx[None] * np.einsum("rbj,bj->rb", code, qx)
    if mo is not None:
        terms = np.concatenate([terms, f16(wb[:, :, mo:mo + 2]) * dx[None] * qx.sum(axis=1)[None]], axis=1)
    return terms


def _k4_scale_min(s, j):
    """get_scale_min_k4 (c:705-714) on scale bytes s [..., 12]."""
    if j < 4:
        return s[..., j] & 63, s[..., j + 4] & 63
    return (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4), (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)


def kquant_magnitudes(qtype, w, rows, cols):
    """Per-element bound [rows, cols] on the magnitudes a factored K-quant dot
    sums: |d*sc| * code + |dmin*m| (Q2_K, Q4_K, Q5_K), |d*s| * (v + 4)
    (Q3_K, code v in 0..7 and offset 4), |d*sc| * (u + 32) (Q6_K)."""
    e, bb = oracle.BLOCK[qtype]
    wb = w.reshape(rows, -1, bb).astype(np.int64)
    A = np.empty((rows, cols // 256, 256))
    if qtype == oracle.Q2_K:
        d, dmin = f16(w.reshape(rows, -1, bb)[:, :, 80:82]), f16(w.reshape(rows, -1, bb)[:, :, 82:84])
        for g in range(16):
            half, j, second = g // 8, (g // 2) % 4, g % 2
            u = (wb[:, :, 16 + 32 * half + 16 * second: 32 + 32 * half + 16 * second] >> (2 * j)) & 3
            sc = wb[:, :, g]
            A[:, :, 16 * g:16 * g + 16] = np.abs(d * (sc & 15))[..., None] * u + np.abs(dmin * (sc >> 4))[..., None]
    elif qtype == oracle.Q3_K:
        d = f16(w.reshape(rows, -1, bb)[:, :, 108:110])
        sb = wb[:, :, 96:108]
        for g in range(16):
            half, j, second = g // 8, (g // 2) % 4, g % 2
            lo = (sb[:, :, g] & 15) if g < 8 else (sb[:, :, g - 8] >> 4)
            s = (lo | (((sb[:, :, 8 + g % 4] >> (2 * (g // 4))) & 3) << 4)) - 32
            u = (wb[:, :, 32 + 32 * half + 16 * second: 48 + 32 * half + 16 * second] >> (2 * j)) & 3
            h = (wb[:, :, 16 * second: 16 * second + 16] >> (4 * half + j)) & 1
            A[:, :, 16 * g:16 * g + 16] = np.abs(d * s)[..., None] * ((u | (h << 2)) + 4)
    elif qtype in (oracle.Q4_K, oracle.Q5_K):
        raw = w.reshape(rows, -1, bb)
        d, dmin = f16(raw[:, :, 0:2]), f16(raw[:, :, 2:4])
        s = wb[:, :, 4:16]
        for k in range(8):
            sc, m = _k4_scale_min(s, k)
            if qtype == oracle.Q4_K:
                q = wb[:, :, 16 + 32 * (k // 2): 48 + 32 * (k // 2)]
                q = (q >> 4) if k % 2 else (q & 15)
            else:
                q = wb[:, :, 48 + 32 * (k // 2): 80 + 32 * (k // 2)]
                q = ((q >> 4) if k % 2 else (q & 15)) + 16 * ((wb[:, :, 16:48] >> k) & 1)
            A[:, :, 32 * k:32 * k + 32] = np.abs(d * sc)[..., None] * q + np.abs(dmin * m)[..., None]
    elif qtype == oracle.Q6_K:
        raw = w.reshape(rows, -1, bb)
        d = f16(raw[:, :, 208:210])
        sc = raw[:, :, 192:208].view(np.int8).astype(np.float64)
        A = np.repeat(np.abs(d[:, :, None] * sc), 16, axis=2) * 95.0
    else:
        raise ValueError(qtype)
    return A.reshape(rows, cols)
