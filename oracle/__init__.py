"""The oracle: a CPU restatement of llama3pure's quantized forward path.

TEST INFRASTRUCTURE.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker.  The product path (``llama3pure_amd``) never imports it.

Two native libraries sit behind it:

* ``_build/libcpuref.so`` — ``cpuref.c``, the restatement (always built);
* ``_ref/libref.so`` — the unmodified reference engine compiled in place by
  ``oracle/Makefile`` (present only where ``/root/reference`` was available at
  build time; tests that need it skip otherwise).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CPUREF_SO = os.path.join(HERE, "_build", "libcpuref.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")
REF_OMP_SO = os.path.join(HERE, "_ref", "libref_omp.so")          # -Ofast -fopenmp -march=x86-64-v3
REF_OMP_V4_SO = os.path.join(HERE, "_ref", "libref_omp_v4.so")    # the same with -march=x86-64-v4 (AVX-512)
REF_SRC = "/root/reference/llama3pure-c-engine.c"

# GGML type ids (llama3pure-c-engine.c:95-113)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, BF16 = 10, 11, 12, 13, 14, 20, 29
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20),
         Q5_0: (32, 22), Q5_1: (32, 24), Q8_0: (32, 34), Q2_K: (256, 84),
         Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
         IQ4_NL: (32, 18)}


def row_bytes(qtype: int, cols: int) -> int:
    e, b = BLOCK[qtype]
    return cols // e * b


def build(with_ref: bool | None = None) -> None:
    """Compile cpuref (always) and the reference harness (when its source exists)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "all"], check=True)
    if with_ref is None:
        with_ref = os.path.exists(REF_SRC)
    if with_ref:
        subprocess.run(["make", "-s", "-B", "-C", HERE, "ref"], check=True)


_F = C.POINTER(C.c_float)
_P = C.c_void_p


def _fp(a):
    return a.ctypes.data_as(_F)


def _vp(a):
    return C.c_void_p(a.ctypes.data)


class _Lib:
    def __init__(self, path, prefix):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = C.CDLL(path)
        self.p = prefix


class CpuRef(_Lib):
    """ctypes view of libcpuref.so (the restatement)."""

    def __init__(self, path: str = CPUREF_SO):
        super().__init__(path, "l3o_")
        L = self.lib
        L.l3o_fp16_to_fp32.restype = C.c_float
        L.l3o_fp16_to_fp32.argtypes = [C.c_uint16]
        L.l3o_fp32_to_fp16.restype = C.c_uint16
        L.l3o_fp32_to_fp16.argtypes = [C.c_float]
        L.l3o_fp16_to_fp32_n.argtypes = [_P, _P, C.c_size_t]
        L.l3o_fp32_to_fp16_n.argtypes = [_P, _P, C.c_size_t]
        L.l3o_dequant_row.argtypes = [C.c_int, _P, _P, C.c_int]
        L.l3o_quantize_q8_0.argtypes = [_P, _P, C.c_int]
        L.l3o_matmul.argtypes = [C.c_int, _P, C.c_int, C.c_int, _P, _P]
        L.l3o_matmul_batch.argtypes = [C.c_int, _P, C.c_int, C.c_int, _P, C.c_int, C.c_int, _P, C.c_int]
        L.l3o_fast_expf.restype = C.c_float
        L.l3o_fast_expf.argtypes = [C.c_float]
        L.l3o_fast_tanhf.restype = C.c_float
        L.l3o_fast_tanhf.argtypes = [C.c_float]
        L.l3o_rmsnorm.argtypes = [_P, _P, _P, C.c_int, C.c_float]
        L.l3o_softmax.argtypes = [_P, C.c_int]
        L.l3o_swiglu.argtypes = [_P, _P, C.c_int]
        L.l3o_geglu.argtypes = [_P, _P, C.c_int]
        L.l3o_rng_u32.restype = C.c_uint32
        L.l3o_rng_u32.argtypes = [C.POINTER(C.c_uint64)]
        L.l3o_rng_f32.restype = C.c_float
        L.l3o_rng_f32.argtypes = [C.POINTER(C.c_uint64)]
        L.l3o_sample.argtypes = [_P, C.c_int, C.c_float, C.c_int, C.c_float, C.POINTER(C.c_uint64)]
        L.l3o_model_open.restype = C.c_void_p
        L.l3o_model_open.argtypes = [_P, C.c_size_t, C.c_int]
        L.l3o_model_close.argtypes = [_P]
        L.l3o_last_error.restype = C.c_char_p
        L.l3o_model_info.argtypes = [_P, _P]
        L.l3o_forward.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P]
        L.l3o_prefill.argtypes = [_P, _P, C.c_int, C.c_int]
        L.l3o_copy_kv.argtypes = [_P, C.c_int, C.c_int, _P, C.c_size_t]
        L.l3o_set_kv.argtypes = [_P, C.c_int, C.c_int, _P, C.c_size_t]
        L.l3o_copy_x.argtypes = [_P, _P]
        L.l3o_rope_row.argtypes = [_P, C.c_int, C.c_int, _P, _P]
        L.l3o_set_attention.argtypes = [_P, C.c_int, C.c_float]
        L.l3o_attend_head.argtypes = [_P, _P, _P, C.c_int, C.c_int, C.c_float, _P, _P]

    # -- primitives --
    def fp16_to_fp32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.l3o_fp16_to_fp32_n(_vp(h), _vp(out), h.size)
        return out

    def fp32_to_fp16(self, f: np.ndarray) -> np.ndarray:
        f = np.ascontiguousarray(f, dtype=np.float32)
        out = np.empty(f.shape, np.uint16)
        self.lib.l3o_fp32_to_fp16_n(_vp(f), _vp(out), f.size)
        return out

    def dequant(self, qtype: int, raw: np.ndarray, n: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.empty(n, np.float32)
        if self.lib.l3o_dequant_row(qtype, _vp(raw), _vp(out), n) != 0:
            raise ValueError(f"unsupported type {qtype}")
        return out

    def quantize_q8_0(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.size // 32 * 34, np.uint8)
        self.lib.l3o_quantize_q8_0(_vp(x), _vp(out), x.size)
        return out

    def matmul(self, qtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, np.float32)
        if self.lib.l3o_matmul(qtype, _vp(w), rows, cols, _vp(x), _vp(y)) != 0:
            raise ValueError(f"unsupported type {qtype}")
        return y

    def matmul_batch(self, qtype, w, rows, cols, x2d):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x2d = np.ascontiguousarray(x2d, dtype=np.float32)
        b = x2d.shape[0]
        y = np.empty((b, rows), np.float32)
        if self.lib.l3o_matmul_batch(qtype, _vp(w), rows, cols, _vp(x2d), b, cols, _vp(y), rows) != 0:
            raise ValueError(f"unsupported type {qtype}")
        return y

    def fast_expf(self, x: float) -> float:
        return self.lib.l3o_fast_expf(x)

    def fast_tanhf(self, x: float) -> float:
        return self.lib.l3o_fast_tanhf(x)

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        o = np.empty_like(x)
        self.lib.l3o_rmsnorm(_vp(o), _vp(x), _vp(w), x.size, eps)
        return o

    def softmax(self, x):
        x = np.array(x, np.float32, copy=True)
        self.lib.l3o_softmax(_vp(x), x.size)
        return x

    def swiglu(self, g, u):
        g = np.array(g, np.float32, copy=True)
        u = np.ascontiguousarray(u, np.float32)
        self.lib.l3o_swiglu(_vp(g), _vp(u), g.size)
        return g

    def geglu(self, g, u):
        g = np.array(g, np.float32, copy=True)
        u = np.ascontiguousarray(u, np.float32)
        self.lib.l3o_geglu(_vp(g), _vp(u), g.size)
        return g

    def attend_head(self, q8, kc, vc, n, hs, cap):
        """One head's attention over n Q8_0 cache rows: (weights, output)."""
        q8, kc, vc = (np.ascontiguousarray(v, np.uint8) for v in (q8, kc, vc))
        att = np.empty(n, np.float32)
        out = np.zeros(hs, np.float32)
        self.lib.l3o_attend_head(_vp(q8), _vp(kc), _vp(vc), n, hs, cap, _vp(att), _vp(out))
        return att, out

    def sample(self, logits, temperature, top_k, top_p, seed):
        """Returns (token, new_seed)."""
        logits = np.ascontiguousarray(logits, np.float32)
        s = C.c_uint64(seed)
        tok = self.lib.l3o_sample(_vp(logits), logits.size, temperature, top_k, top_p, C.byref(s))
        return tok, s.value

    def rng_u32(self, seed, n):
        s = C.c_uint64(seed)
        return [self.lib.l3o_rng_u32(C.byref(s)) for _ in range(n)]

    def open_model(self, gguf: bytes, context_size: int = 0) -> "CpuModel":
        return CpuModel(self, gguf, context_size)


class CpuModel:
    """A model in the restatement: forward/prefill with reference arithmetic."""

    def __init__(self, ref: CpuRef, gguf: bytes, context_size: int):
        self.ref = ref
        # a uint8 array is borrowed as is (multi-GB images are not copied);
        # bytes are copied into an array the model keeps alive
        if isinstance(gguf, np.ndarray) and gguf.dtype == np.uint8 and gguf.flags.c_contiguous:
            self._buf = gguf
        else:
            self._buf = np.frombuffer(gguf, dtype=np.uint8).copy()
        h = ref.lib.l3o_model_open(_vp(self._buf), self._buf.size, context_size)
        if not h:
            raise ValueError(ref.lib.l3o_last_error().decode())
        self.h = C.c_void_p(h)
        info = np.zeros(11, np.int32)
        ref.lib.l3o_model_info(self.h, _vp(info))
        (self.dim, self.hidden, self.n_layers, self.n_heads, self.n_kv, self.vocab,
         self.seq_len, self.head_dim, self.is_gemma, self.swa_window, self.swa_pattern) = map(int, info)

    def forward(self, token: int, pos: int, logits: bool = True):
        out = np.empty(self.vocab, np.float32)
        rc = self.ref.lib.l3o_forward(self.h, token, pos, int(logits), _vp(out))
        if rc != 0:
            raise RuntimeError(f"l3o_forward rc={rc}")
        return out if logits else None

    def prefill(self, tokens, start: int, bs: int):
        t = np.ascontiguousarray(tokens, np.int32)
        rc = self.ref.lib.l3o_prefill(self.h, _vp(t), start, bs)
        if rc != 0:
            raise RuntimeError(f"l3o_prefill rc={rc}")

    def kv(self, layer: int, which_v: bool) -> np.ndarray:
        n = self.n_kv * self.seq_len * (self.head_dim // 32 * 34)
        out = np.empty(n, np.uint8)
        if self.ref.lib.l3o_copy_kv(self.h, layer, int(which_v), _vp(out), n) != 0:
            raise RuntimeError("copy_kv")
        return out

    def set_attention(self, swa_pattern: int = 0, attn_softcap: float = 0.0) -> None:
        """The load options the reference lacks: a sliding-window layer
        pattern (0 keeps the model's) and an attention score cap (0: none)."""
        if self.ref.lib.l3o_set_attention(self.h, swa_pattern, attn_softcap) != 0:
            raise ValueError("set_attention")

    def set_kv(self, layer: int, which_v: bool, data: np.ndarray) -> None:
        """Overwrite one layer's K or V cache (test support: installs a long
        context without prefilling it in the oracle)."""
        data = np.ascontiguousarray(data, np.uint8)
        if self.ref.lib.l3o_set_kv(self.h, layer, int(which_v), _vp(data), data.size) != 0:
            raise RuntimeError("set_kv")

    def rope_row(self, swa: bool, pos: int):
        c = np.empty(self.head_dim // 2, np.float32)
        s = np.empty(self.head_dim // 2, np.float32)
        if self.ref.lib.l3o_rope_row(self.h, int(swa), pos, _vp(c), _vp(s)) != 0:
            raise RuntimeError("rope_row")
        return c, s

    def x(self) -> np.ndarray:
        out = np.empty(self.dim, np.float32)
        self.ref.lib.l3o_copy_x(self.h, _vp(out))
        return out

    def close(self):
        if self.h:
            self.ref.lib.l3o_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Ref(_Lib):
    """ctypes view of _ref/libref.so: the reference engine itself.

    The reference keeps its model in process globals, so one process can hold
    one reference model at a time (tests run it in a subprocess when needed).
    """

    def __init__(self, path: str = REF_SO):
        super().__init__(path, "ref_")
        L = self.lib
        L.ref_fp16_to_fp32.restype = C.c_float
        L.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        L.ref_fp32_to_fp16.restype = C.c_uint16
        L.ref_fp32_to_fp16.argtypes = [C.c_float]
        L.ref_fp16_to_fp32_n.argtypes = [_P, _P, C.c_size_t]
        L.ref_fp32_to_fp16_n.argtypes = [_P, _P, C.c_size_t]
        L.ref_dequant_row.argtypes = [C.c_int, _P, _P, C.c_int]
        L.ref_quantize_q8_0.argtypes = [_P, _P, C.c_int]
        L.ref_matmul.argtypes = [C.c_int, _P, C.c_int, C.c_int, _P, _P]
        L.ref_matmul_batch.argtypes = [C.c_int, _P, C.c_int, C.c_int, _P, C.c_int, C.c_int, _P, C.c_int]
        L.ref_fast_expf.restype = C.c_float
        L.ref_fast_expf.argtypes = [C.c_float]
        L.ref_fast_tanhf.restype = C.c_float
        L.ref_fast_tanhf.argtypes = [C.c_float]
        L.ref_rmsnorm.argtypes = [_P, _P, _P, C.c_int, C.c_float]
        L.ref_softmax.argtypes = [_P, C.c_int]
        L.ref_model_open.argtypes = [C.c_char_p, C.c_int]
        L.ref_forward.argtypes = [C.c_int, C.c_int, C.c_int, _P]
        L.ref_prefill.argtypes = [_P, C.c_int, C.c_int]
        L.ref_copy_kv.argtypes = [C.c_int, C.c_int, _P, C.c_size_t]
        L.ref_set_kv.argtypes = [C.c_int, C.c_int, _P, C.c_size_t]
        L.ref_copy_x.argtypes = [_P]
        L.ref_rope_row.argtypes = [C.c_int, C.c_int, _P, _P]
        L.ref_generate_token.argtypes = [C.c_int, C.c_int, C.c_float, C.c_int, C.c_float, C.POINTER(C.c_ulonglong)]
        L.ref_init()

    def fp16_to_fp32(self, h):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.ref_fp16_to_fp32_n(_vp(h), _vp(out), h.size)
        return out

    def fp32_to_fp16(self, f):
        f = np.ascontiguousarray(f, np.float32)
        out = np.empty(f.shape, np.uint16)
        self.lib.ref_fp32_to_fp16_n(_vp(f), _vp(out), f.size)
        return out

    def dequant(self, qtype, raw, n):
        raw = np.ascontiguousarray(raw, np.uint8)
        out = np.empty(n, np.float32)
        self.lib.ref_dequant_row(qtype, _vp(raw), _vp(out), n)
        return out

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.size // 32 * 34, np.uint8)
        self.lib.ref_quantize_q8_0(_vp(x), _vp(out), x.size)
        return out

    def matmul(self, qtype, w, rows, cols, x):
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        self.lib.ref_matmul(qtype, _vp(w), rows, cols, _vp(x), _vp(y))
        return y

    def matmul_batch(self, qtype, w, rows, cols, x2d):
        w = np.ascontiguousarray(w, np.uint8)
        x2d = np.ascontiguousarray(x2d, np.float32)
        b = x2d.shape[0]
        y = np.empty((b, rows), np.float32)
        self.lib.ref_matmul_batch(qtype, _vp(w), rows, cols, _vp(x2d), b, cols, _vp(y), rows)
        return y

    def rmsnorm(self, x, w, eps):
        x = np.array(x, np.float32, copy=True)
        w = np.array(w, np.float32, copy=True)
        o = np.empty_like(x)
        self.lib.ref_rmsnorm(_vp(o), _vp(x), _vp(w), x.size, eps)
        return o

    def softmax(self, x):
        x = np.array(x, np.float32, copy=True)
        self.lib.ref_softmax(_vp(x), x.size)
        return x


def have_ref() -> bool:
    return os.path.exists(REF_SO)
