"""llama3pure_amd — MI355X-native quantized forward path of llama3pure.

The product is ``libl3p.so`` (HIP kernels for gfx950 behind the C-ABI in
``include/l3p.h``).  This module is a thin ctypes view of that library for
Python callers (tests, ``bench.py``); Node.js callers use the N-API addon in
``js/``.  There is no CPU fallback: if the library is missing, importing
:func:`lib` raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libl3p.so")

# GGML type ids (llama3pure-c-engine.c:95-113)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, BF16 = 10, 11, 12, 13, 14, 20, 29

OK = 0
E_INVALID, E_UNSUPPORTED, E_HIP, E_NOMEM, E_FORMAT, E_STATE = -1, -2, -3, -4, -5, -6

EXPORTS = [
    "l3p_create", "l3p_destroy", "l3p_last_error", "l3p_stream", "l3p_synchronize",
    "l3p_malloc", "l3p_free", "l3p_upload", "l3p_download", "l3p_row_bytes",
    "l3p_dequant", "l3p_quantize_q8_0", "l3p_gemv", "l3p_gemm",
    "l3p_load_gguf", "l3p_get_model_info", "l3p_forward", "l3p_prefill", "l3p_decode", "l3p_generate_greedy",
    "l3p_sample", "l3p_logits_device", "l3p_copy_kv", "l3p_rope_row",
    "l3p_profile", "l3p_profile_read", "l3p_stream_read", "l3p_gemm_static", "l3p_generate_sampled",
]


class L3PError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"l3p error {code}: {msg}")
        self.code = code


class LoadOpts(C.Structure):
    _fields_ = [("context_size", C.c_int), ("swa_pattern", C.c_int), ("attn_softcap", C.c_float),
                ("reserved", C.c_int * 5)]


class ModelInfo(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                                       "vocab_size", "seq_len", "head_dim", "is_gemma", "swa_window",
                                       "swa_pattern", "weight_type")] + \
               [(n, C.c_float) for n in ("rope_theta", "rope_theta_swa", "rms_eps", "final_softcap")] + \
               [("device_bytes", C.c_int64), ("attn_softcap", C.c_float), ("reserved", C.c_int)]


class KernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("launches", C.c_int64), ("total_ms", C.c_double),
                ("bytes_per_launch", C.c_double), ("p10_ms", C.c_double), ("p50_ms", C.c_double),
                ("p90_ms", C.c_double)]


class Sampler(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("reserved", C.c_int)]


_lib = None


def lib() -> C.CDLL:
    """Load libl3p.so (built by ``python -m llama3pure_amd.build``)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m llama3pure_amd.build`")
    L = C.CDLL(LIB_PATH)
    P, I, I64, SZ = C.c_void_p, C.c_int, C.c_int64, C.c_size_t
    sig = {
        "l3p_create": (I, [I, C.POINTER(P)]),
        "l3p_destroy": (None, [P]),
        "l3p_last_error": (C.c_char_p, [P]),
        "l3p_stream": (P, [P]),
        "l3p_synchronize": (I, [P]),
        "l3p_malloc": (I, [P, SZ, C.POINTER(P)]),
        "l3p_free": (I, [P, P]),
        "l3p_upload": (I, [P, P, P, SZ]),
        "l3p_download": (I, [P, P, P, SZ]),
        "l3p_row_bytes": (SZ, [I, I]),
        "l3p_dequant": (I, [P, I, P, I64, P]),
        "l3p_quantize_q8_0": (I, [P, P, I64, P]),
        "l3p_gemv": (I, [P, I, P, I, I, P, P]),
        "l3p_gemm": (I, [P, I, P, I, I, P, I, I, P, I]),
        "l3p_load_gguf": (I, [P, P, SZ, C.POINTER(LoadOpts)]),
        "l3p_get_model_info": (I, [P, C.POINTER(ModelInfo)]),
        "l3p_forward": (I, [P, C.c_int32, C.c_int32, I, P]),
        "l3p_prefill": (I, [P, P, I, C.c_int32]),
        "l3p_decode": (I, [P, C.c_int32, C.c_int32, C.POINTER(Sampler), C.POINTER(C.c_uint64),
                           C.POINTER(C.c_int32)]),
        "l3p_generate_greedy": (I, [P, C.c_int32, C.c_int32, C.c_int32, P, C.c_int32, P, C.POINTER(C.c_int32)]),
        "l3p_sample": (I, [P, P, I, C.POINTER(Sampler), C.POINTER(C.c_uint64), C.POINTER(C.c_int32)]),
        "l3p_logits_device": (I, [P, C.POINTER(P)]),
        "l3p_copy_kv": (I, [P, I, I, P, SZ]),
        "l3p_rope_row": (I, [P, I, I, P, P]),
        "l3p_profile": (I, [P, I]),
        "l3p_profile_read": (I, [P, C.POINTER(KernelStat), I, C.POINTER(I)]),
        "l3p_stream_read": (I, [P, P, C.c_size_t]),
        "l3p_gemm_static": (I, [I, P, I, I, P, I, I, P, I, P]),
        "l3p_generate_sampled": (I, [P, C.c_int32, C.c_int32, C.c_int32, C.POINTER(Sampler), C.POINTER(C.c_uint64),
                                     P, C.c_int32, P, C.POINTER(C.c_int32)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def row_bytes(qtype: int, cols: int) -> int:
    return int(lib().l3p_row_bytes(qtype, cols))


def _ptr(x) -> int:
    """Device or host address of a torch tensor / numpy array / int."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError(type(x))


class Context:
    """One l3p context (device + stream + optional model)."""

    def __init__(self, device: int = 0):
        self.L = lib()
        h = C.c_void_p()
        rc = self.L.l3p_create(device, C.byref(h))
        if rc != OK:
            raise L3PError(rc, self.L.l3p_last_error(None).decode())
        self.h = h

    # -- plumbing --
    def _check(self, rc: int):
        if rc != OK:
            raise L3PError(rc, self.L.l3p_last_error(self.h).decode())

    @property
    def stream(self) -> int:
        return self.L.l3p_stream(self.h)

    def synchronize(self):
        self._check(self.L.l3p_synchronize(self.h))

    def close(self):
        if getattr(self, "h", None):
            self.L.l3p_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- ops (device pointers) --
    def gemv(self, qtype, w, rows, cols, x, y):
        self._check(self.L.l3p_gemv(self.h, qtype, _ptr(w), rows, cols, _ptr(x), _ptr(y)))

    def gemm(self, qtype, w, rows, cols, x, batch, in_stride, y, out_stride):
        self._check(self.L.l3p_gemm(self.h, qtype, _ptr(w), rows, cols, _ptr(x), batch, in_stride,
                                    _ptr(y), out_stride))

    def dequant(self, qtype, src, n, dst):
        self._check(self.L.l3p_dequant(self.h, qtype, _ptr(src), n, _ptr(dst)))

    def quantize_q8_0(self, x, n, dst):
        self._check(self.L.l3p_quantize_q8_0(self.h, _ptr(x), n, _ptr(dst)))

    # -- model --
    def load_gguf(self, gguf, context_size: int = 0, swa_pattern: int = 0, attn_softcap: float = 0.0):
        import numpy as np
        buf = gguf if isinstance(gguf, np.ndarray) else np.frombuffer(gguf, dtype=np.uint8)
        opts = LoadOpts(context_size=context_size, swa_pattern=swa_pattern, attn_softcap=attn_softcap)
        self._check(self.L.l3p_load_gguf(self.h, buf.ctypes.data, buf.nbytes, C.byref(opts)))
        return self.model_info()

    def model_info(self) -> ModelInfo:
        mi = ModelInfo()
        self._check(self.L.l3p_get_model_info(self.h, C.byref(mi)))
        return mi

    def forward(self, token: int, pos: int, logits: bool = True):
        import numpy as np
        out = None
        if logits:
            out = np.empty(self.model_info().vocab_size, np.float32)
        self._check(self.L.l3p_forward(self.h, token, pos, int(logits), _ptr(out)))
        return out

    def prefill(self, tokens, start: int):
        import numpy as np
        t = np.ascontiguousarray(tokens, np.int32)
        self._check(self.L.l3p_prefill(self.h, t.ctypes.data, t.size, start))

    def decode(self, token: int, pos: int, temperature=0.0, top_k=40, top_p=0.9, rng: int = 0):
        """Returns (next_token, new_rng_state)."""
        s = Sampler(temperature, top_k, top_p, 0)
        st = C.c_uint64(rng)
        out = C.c_int32()
        self._check(self.L.l3p_decode(self.h, token, pos, C.byref(s), C.byref(st), C.byref(out)))
        return out.value, st.value

    def generate_greedy(self, token: int, pos: int, max_steps: int, stop_ids=()):
        """Greedy tokens of up to max_steps steps from (token, pos), ending
        after the first stop id (included); queued ahead on the device."""
        import numpy as np
        stops = np.ascontiguousarray(stop_ids, np.int32)
        out = np.zeros(max(1, max_steps), np.int32)
        n = C.c_int32()
        self._check(self.L.l3p_generate_greedy(self.h, token, pos, max_steps, stops.ctypes.data if stops.size else None,
                                               stops.size, out.ctypes.data, C.byref(n)))
        return out[:n.value].tolist()

    def generate_sampled(self, token: int, pos: int, max_steps: int, temperature=0.9, top_k=40, top_p=0.9,
                         rng: int = 0, stop_ids=()):
        """Sampled tokens of up to max_steps steps from (token, pos), ending
        after the first stop id (included), and the final RNG state; queued
        ahead on the device, the sampler finished on the host per step."""
        import numpy as np
        stops = np.ascontiguousarray(stop_ids, np.int32)
        out = np.zeros(max(1, max_steps), np.int32)
        n = C.c_int32()
        s = Sampler(temperature, top_k, top_p, 0)
        st = C.c_uint64(rng)
        self._check(self.L.l3p_generate_sampled(self.h, token, pos, max_steps, C.byref(s), C.byref(st),
                                                stops.ctypes.data if stops.size else None, stops.size,
                                                out.ctypes.data, C.byref(n)))
        return out[:n.value].tolist(), st.value

    def sample(self, logits_dev, n, temperature=0.0, top_k=40, top_p=0.9, rng: int = 0):
        s = Sampler(temperature, top_k, top_p, 0)
        st = C.c_uint64(rng)
        out = C.c_int32()
        self._check(self.L.l3p_sample(self.h, _ptr(logits_dev), n, C.byref(s), C.byref(st), C.byref(out)))
        return out.value, st.value

    def logits(self):
        """The vocab logits of the last step run (forward, decode, or the step
        generate_greedy queued past a stop), copied from the device."""
        import numpy as np
        d = C.c_void_p()
        self._check(self.L.l3p_logits_device(self.h, C.byref(d)))
        out = np.empty(self.model_info().vocab_size, np.float32)
        self._check(self.L.l3p_download(self.h, out.ctypes.data, d, out.nbytes))
        return out

    def copy_kv(self, layer: int, which_v: bool):
        import numpy as np
        mi = self.model_info()
        n = mi.n_kv_heads * mi.seq_len * (mi.head_dim // 32 * 34)
        out = np.empty(n, np.uint8)
        self._check(self.L.l3p_copy_kv(self.h, layer, int(which_v), out.ctypes.data, n))
        return out

    def profile(self, on: bool):
        """Start (clearing earlier figures) or stop GEMV launch timing."""
        self._check(self.L.l3p_profile(self.h, int(on)))

    def _profile_stats(self):
        n = C.c_int(0)
        self._check(self.L.l3p_profile_read(self.h, None, 0, C.byref(n)))
        arr = (KernelStat * max(1, n.value))()
        self._check(self.L.l3p_profile_read(self.h, arr, n.value, C.byref(n)))
        return [arr[i] for i in range(n.value)]

    def profile_read(self):
        """{label: (launches, total_ms, algorithmic bytes per launch)} of the timed GEMV launches."""
        return {s.name.decode(): (s.launches, s.total_ms, s.bytes_per_launch) for s in self._profile_stats()}

    def stream_read(self, buf, nbytes: int):
        """A plain streaming read of nbytes of the device buffer (timed under profile())."""
        self._check(self.L.l3p_stream_read(self.h, _ptr(buf), nbytes))

    def profile_percentiles(self):
        """{label: (p10_ms, p50_ms, p90_ms)} of the timed launches' durations."""
        return {s.name.decode(): (s.p10_ms, s.p50_ms, s.p90_ms) for s in self._profile_stats()}

    def rope_row(self, swa: bool, pos: int):
        import numpy as np
        half = self.model_info().head_dim // 2
        c = np.empty(half, np.float32)
        s = np.empty(half, np.float32)
        self._check(self.L.l3p_rope_row(self.h, int(swa), pos, c.ctypes.data, s.ctypes.data))
        return c, s
