"""Decode throughput of the quantized forward path on one MI355X.

Workload (one "step" = one greedy decode token, forward + on-device sampling,
only the token id returns to the host): a random-init Llama-3-8B-architecture
model, every matrix Q8_0 (32 layers, dim 4096, 32 query / 8 KV heads, head_dim
128, SwiGLU 14336, vocab 128256, RoPE theta 500000, RMSNorm eps 1e-5, weights
N(0, 0.02) before quantization, norm weights 1.0), KV cache prefilled to
position 1024 of a 2048 context with uniform random token ids.

Printed as one JSON line:
  value        decode tok/s over exactly --steps timed steps (weights, KV
               cache and run state already resident in HBM), run as the
               reference's greedy loop through l3p_generate_greedy (each
               step's token read back while the next step runs);
               per_call_decode times the same number of steps as one
               synchronous l3p_decode call per token;
  roofline     the dominant GEMV launch class: algorithmic bytes per launch
               over its average kernel duration, from the HIP events each
               GEMV dispatch records at its own start and end
               (hipExtLaunchKernelGGL), over a second pass of --steps decode
               steps (run eagerly);
  gemv         standalone GEMV launches at the Llama-3-8B shapes (Q8_0, Q4_0,
               Q4_K, Q6_K), timed the same way, weight copies rotated through
               >= 1 GiB so the 256 MB last-level cache does not serve them;
  prefill      the 1024-position prompt before the decode: positions/s and
               the fp32-MFMA roofline of the dominant prefill GEMM class;
  cpu_baseline the reference C engine (oracle/_ref/libref_omp.so: its own
               source built with its Makefile's -Ofast -fopenmp line) decoding
               the same GGUF on the host at positions 1024.. for a bounded
               sample, with the threads this process is given
               (OMP_NUM_THREADS, else its affinity mask; nproc and the lscpu
               model are recorded), and its basic -O3 build on one thread
               (single_thread_O3); the oracle (C restatement) when the
               reference is not built.

usage: python bench.py [--gpus 1] [--steps 128] [--warmup 8]

Measurement-only modes (one JSON line per case, no decode): --gemv-shapes,
--gemm-types (the batched product of every weight type at 4096 x 4096 x 1024
rows), --prefill-types (a 1024-position prompt through four
Llama-3-8B-shape layers for several weight mixes), --attn-sweep,
--copy-ceiling, --calibrate-copy.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0   # MI355X HBM3E, 8 TB/s
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix peak
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_decode_gemv.md")

LLAMA3_8B = dict(arch="llama", dim=4096, hidden=14336, n_layers=32, n_heads=32, n_kv=8, vocab=128256, ctx=2048,
                 rope_theta=500000.0, eps=1e-5, std=0.02, seed=1234)


# Gemma-2-2B dimensions on the reference's Gemma path (QK-norm, post norms,
# NEOX RoPE, GeGLU, tied embedding, final logit soft-cap 30); the 4096-position
# local window covers the whole 1024-position context, as in Gemma-2 at this
# length.  Attention soft-capping is in neither reference engine.
GEMMA2_2B = dict(arch="gemma3", dim=2304, hidden=9216, n_layers=26, n_heads=8, n_kv=4, head_dim=256, vocab=256000,
                 ctx=1024, softcap=30.0, swa_window=4096, tied=True, rope_theta=10000.0, eps=1e-6, std=0.02,
                 seed=4321)
# the workload's Gemma-2 attention: alternating local/global layers and the
# attention score cap 50 (load options; see gemma_prompt_decode)
GEMMA2_2B_LOAD = dict(swa_pattern=2, attn_softcap=50.0)


def time_gemv_shapes(ctx, torch, l3p, synth):
    """GB/s of single GEMV launches: at least 200 l3p_gemv calls over rotating
    weight copies (>= 1 GiB, so no launch finds its weights in a cache), each
    kernel timed by its own dispatch events (the library's launch timing);
    mean and p10/p50/p90 of the launch durations."""
    shapes = [("q8_0", l3p.Q8_0, 4096, 4096), ("q4_0", l3p.Q4_0, 14336, 4096), ("q4_0", l3p.Q4_0, 4096, 14336),
              ("q4_k", l3p.Q4_K, 14336, 4096), ("q6_k", l3p.Q6_K, 128256, 4096)]
    out = []
    for name, qt, rows, cols in shapes:
        wbytes = rows * synth.row_bytes(qt, cols)
        copies = max(2, -(-(1 << 30) // wbytes))
        base = torch.from_numpy(synth.random_blocks(qt, rows, cols, seed=7)).cuda()
        ws = [base.clone() for _ in range(copies)]
        x = torch.from_numpy(synth.random_x(cols, seed=8)).cuda()
        y = torch.empty(rows, device="cuda")
        torch.cuda.synchronize()
        for i in range(copies):
            ctx.gemv(qt, ws[i], rows, cols, x, y)
        ctx.synchronize()
        n = max(200, 2 * copies)
        ctx.profile(True)
        for i in range(n):
            ctx.gemv(qt, ws[i % copies], rows, cols, x, y)
        stats = ctx.profile_read()
        p10, p50, p90 = next(iter(ctx.profile_percentiles().values()))
        ctx.profile(False)
        launches, ms, _ = next(iter(stats.values()))
        avg = ms * 1e3 / launches
        alg = wbytes + 4 * cols + 4 * rows
        out.append({"shape": f"{name} {rows}x{cols}", "launches": launches, "us": round(avg, 2),
                    "GB/s": round(alg / avg / 1e3, 1), "frac": round(alg / avg / 1e3 / HBM_PEAK_GBS, 4),
                    "us_p10_p50_p90": [round(p10 * 1e3, 2), round(p50 * 1e3, 2), round(p90 * 1e3, 2)]})
        del ws, base
        torch.cuda.empty_cache()
    return out


def prefill_summary(positions: int, seconds: float, stats: dict) -> dict:
    """Prompt throughput and the fp32-MFMA roofline of the dominant GEMM class
    (labels "<type> gemm <what> <N>x<K> b<rows>", 2*N*K*rows flops a launch)."""
    gemms = {k: v for k, v in stats.items() if " gemm " in k}
    out = {"positions": positions, "ms": round(seconds * 1e3, 2), "tok_s": round(positions / seconds, 1)}
    if not gemms:
        return out
    name, (launches, ms, _) = max(gemms.items(), key=lambda kv: kv[1][1])
    n, k = (int(v) for v in name.split()[3].split("x"))
    rows = int(name.split()[4][1:])
    flops = 2.0 * n * k * rows
    avg_us = ms * 1e3 / launches
    tf = flops / (avg_us * 1e-6) / 1e12
    out["gemm_ms"] = round(sum(v[1] for v in gemms.values()), 2)
    out["roofline"] = {"bound": "mfma", "kernel": name, "achieved": round(tf, 1), "peak": MFMA_F32_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": round(tf / MFMA_F32_PEAK_TFLOPS, 4), "flops_per_launch": flops,
                       "avg_launch_us": round(avg_us, 2), "launches": launches}
    return out


def gemma_prompt_decode(np, torch, l3p, synth, prompt_len=512, steps=128, warmup=4):
    """A 512-token prompt, then 128 sampled decode steps (temperature 0.9,
    top-k 40, top-p 0.9, fixed seed) on a random-init Gemma-2-2B-architecture
    Q8_0 model, loaded with Gemma-2's attention: alternating local/global
    layers (swa_pattern 2, window 4096) and the attention score cap 50, next
    to the final logit cap 30.  The prompt is run once untimed (settling
    launch configurations) with `warmup` decode steps after it, then timed;
    the decode steps then continue from the timed prompt as one
    l3p_generate_sampled call (steps queued on the device ahead of the host,
    which finishes each step's sampler in the reference's arithmetic and hands
    the token back through pinned memory); `per_call_decode` times the same
    steps as one synchronous l3p_decode call per token."""
    ctx = l3p.Context(0)
    img = synth.synthetic_model(qtype=synth.Q8_0, make_mat=synth.gpu_q8_0_maker(ctx, torch, 77), **GEMMA2_2B)
    mi = ctx.load_gguf(img, **GEMMA2_2B_LOAD)
    del img
    prompt = np.random.default_rng(6).integers(0, mi.vocab_size, prompt_len).astype(np.int32)
    sampler = dict(temperature=0.9, top_k=40, top_p=0.9)

    def run(n, tok, pos, rng):
        for _ in range(n):
            tok, rng = ctx.decode(tok, pos, rng=rng, **sampler)
            pos += 1
        return tok, pos, rng

    ctx.prefill(prompt[:-1], 0)
    run(warmup, int(prompt[-1]), prompt_len - 1, 42)
    ctx.generate_sampled(int(prompt[-1]), prompt_len - 1, warmup, rng=42, **sampler)
    ctx.synchronize()
    t0 = time.perf_counter()
    ctx.prefill(prompt[:-1], 0)
    ctx.synchronize()
    t_pre = time.perf_counter() - t0
    t0 = time.perf_counter()
    toks, rng = ctx.generate_sampled(int(prompt[-1]), prompt_len - 1, steps, rng=42, **sampler)
    ctx.synchronize()
    t_dec = time.perf_counter() - t0
    tok = toks[-1]
    t0 = time.perf_counter()
    tok_c, _, rng_c = run(steps, int(prompt[-1]), prompt_len - 1, 42)
    ctx.synchronize()
    t_call = time.perf_counter() - t0
    assert (tok_c, rng_c) == (tok, rng), "queued and per-call sampled decode disagree"
    ctx.profile(True)
    ctx.prefill(prompt[:-1], 0)
    pstats = ctx.profile_read()
    ctx.profile(False)
    ctx.close()
    pre = prefill_summary(prompt_len - 1, t_pre, pstats)
    return {"workload": "Gemma-2-2B architecture, all matrices Q8_0: 512-token prompt, then 128 decode steps "
                        "sampled at temperature 0.9, top-k 40, top-p 0.9; load options swa_pattern 2 "
                        "(alternating local window-4096 / global layers) and attn_softcap 50, final logit "
                        "soft-cap 30 from the GGUF",
            "layers": 26, "dim": 2304, "heads": 8, "kv_heads": 4, "head_dim": 256, "ffn": 9216, "vocab": 256000,
            "prefill": pre, "decode_steps": steps, "decode_ms": round(t_dec * 1e3, 2),
            "decode_tok_s": round(steps / t_dec, 1), "last_token": int(tok),
            "per_call_decode": {"call": "l3p_decode once per token from Python (synchronous)",
                                "tok_s": round(steps / t_call, 1)}}


def read_ceiling(ctx, torch, nbytes: int) -> float:
    """GB/s of a plain streaming read of nbytes (l3p_stream_read: nontemporal
    16-byte loads, four in flight per thread): buffers rotated through >= 1
    GiB so the 256 MB MALL does not serve them, each read timed by its own
    dispatch events; the median of at least 40 reads."""
    nbytes = nbytes // 16 * 16
    copies = max(2, -(-(1 << 30) // nbytes))
    bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(copies)]
    torch.cuda.synchronize()
    for b in bufs:
        ctx.stream_read(b, nbytes)
    ctx.synchronize()
    ctx.profile(True)
    for i in range(max(40, 2 * copies)):
        ctx.stream_read(bufs[i % copies], nbytes)
    p50 = next(iter(ctx.profile_percentiles().values()))[1]
    ctx.profile(False)
    del bufs
    torch.cuda.empty_cache()
    return nbytes / (p50 * 1e-3) / 1e9


def gemv_shapes_only():
    """The standalone GEMV lines, then the streaming-read ceiling at each
    shape's weight bytes, in that order (a kernel trace takes the last 200
    GEMV dispatches of each kernel and each block of stream_read_kernel
    dispatches in turn)."""
    import torch

    import llama3pure_amd as l3p
    from llama3pure_amd import synth

    ctx = l3p.Context(0)
    gemv = time_gemv_shapes(ctx, torch, l3p, synth)
    for g in gemv:
        name, shape = g["shape"].split()
        rows, cols = (int(v) for v in shape.split("x"))
        nbytes = rows * synth.row_bytes({"q8_0": l3p.Q8_0, "q4_0": l3p.Q4_0, "q4_k": l3p.Q4_K,
                                         "q6_k": l3p.Q6_K}[name], cols)
        g["read_ceiling_GBps"] = round(read_ceiling(ctx, torch, nbytes), 1)
        g["frac_of_read_ceiling"] = round(g["GB/s"] / g["read_ceiling_GBps"], 4)
        print(json.dumps(g), flush=True)
    ctx.close()


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE +
    WRITE_SIZE summary (a line "traffic <kernel>: <bytes>"), else None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith(f"traffic {kernel}:"):
                    return int(float(line.split(":")[1]))
    except OSError:
        pass
    return None


def calibrate_copy():
    """512 MiB device-to-device copies: FETCH_SIZE and WRITE_SIZE per copy
    dispatch should each read 524288 KiB; the ratio scales the GEMV counts."""
    import torch
    a = torch.empty(1 << 27, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1.0)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": a.numel() * 4, "copies": 5}), flush=True)


def copy_ceiling():
    """An independent check of the streaming-read ceiling: at each size (the
    Q8_0 4096 x 4096 weights, the 4-bit FFN shapes' weights, the Llama-3-8B
    gate|up pair's, and 512 MiB) the runtime's device-to-device copy and
    l3p_stream_read, each over buffers rotated through >= 1 GiB so the 256 MB
    last-level cache serves none of them, each launch timed by its own
    events; the median of >= 40 launches.  The copy reads N and writes N
    bytes: its read side runs at N / t (the counters FETCH_SIZE and
    WRITE_SIZE of the same run give the bytes each copy dispatch moves)."""
    import torch

    import llama3pure_amd as l3p

    ctx = l3p.Context(0)
    sizes = [("q8_0 4096x4096 weights", 4096 * 4352), ("q4_0 14336x4096 weights", 14336 * 2304),
             ("q8_0 gate|up 28672x4096 weights", 28672 * 4352), ("512 MiB", 512 << 20)]
    for name, nbytes in sizes:
        nbytes = nbytes // 16 * 16
        copies = max(2, -(-(1 << 30) // nbytes))
        src = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(copies)]
        dst = [torch.empty_like(src[0]) for _ in range(2)]
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        ts = []
        for i in range(max(40, 2 * copies) + copies):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(st)
            dst[i % 2].copy_(src[i % copies])
            b.record(st)
            ts.append((a, b))
        torch.cuda.synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 for a, b in ts[copies:])
        t_copy = us[len(us) // 2]
        del dst
        for b in src:
            ctx.stream_read(b, nbytes)
        ctx.synchronize()
        ctx.profile(True)
        for i in range(max(40, 2 * copies)):
            ctx.stream_read(src[i % copies], nbytes)
        t_read = next(iter(ctx.profile_percentiles().values()))[1] * 1e3
        ctx.profile(False)
        del src
        torch.cuda.empty_cache()
        print(json.dumps({"bytes": nbytes, "what": name, "copy_us": round(t_copy, 2),
                          "copy_read_side_GBps": round(nbytes / t_copy / 1e3, 1),
                          "copy_total_GBps": round(2 * nbytes / t_copy / 1e3, 1),
                          "stream_read_us": round(t_read, 2), "stream_read_GBps": round(nbytes / t_read / 1e3, 1)}),
              flush=True)
    ctx.close()


def attn_sweep(shape: str):
    """Both decode attentions at several context lengths, for a kernel trace:
    a 2-layer model with the attention of Llama-3-8B (32 query / 8 KV heads,
    head_dim 128) or Gemma-2-2B (8 query / 4 KV heads, head_dim 256, QK-norm),
    4096 positions; per length P, P prompt positions, then 12 decode steps at
    position P with the per-head kernel (L3P_ATTN_HEAD=1) and 12 with chunks +
    merge (=0).  Prints the order of the blocks; the kernel durations come
    from the trace."""
    import numpy as np
    import torch

    import llama3pure_amd as l3p
    from llama3pure_amd import synth

    ctx = l3p.Context(0)
    if shape == "gemma2b":
        g = synth.synthetic_model(arch="gemma3", dim=2304, hidden=256, n_layers=2, n_heads=8, n_kv=4, head_dim=256,
                                  vocab=256, ctx=4096, softcap=30.0, swa_window=4096, tied=True, seed=3)
    else:
        g = synth.synthetic_model(arch="llama", dim=4096, hidden=256, n_layers=2, n_heads=32, n_kv=8, vocab=256,
                                  ctx=4096, seed=3)
    ctx.load_gguf(g)
    toks = np.random.default_rng(1).integers(0, 256, 4096).astype(np.int32)
    order = []
    for P in (64, 256, 512, 640, 1024, 2048, 3000):
        ctx.prefill(toks[:P], 0)
        for path in ("0", "1"):
            os.environ["L3P_ATTN_HEAD"] = path
            for _ in range(12):
                ctx.forward(int(toks[P]), P, logits=False)
            ctx.synchronize()
            order.append({"positions": P + 1, "attention": "per-head" if path == "1" else "chunks+merge"})
    os.environ.pop("L3P_ATTN_HEAD", None)
    torch.cuda.synchronize()
    print(json.dumps({"attn_sweep": order}), flush=True)
    ctx.close()


GEMV_SHAPES = [("q8_0", 8, 4096, 4096), ("q4_0", 2, 14336, 4096), ("q4_0", 2, 4096, 14336), ("q4_k", 12, 14336, 4096),
               ("q6_k", 14, 128256, 4096)]   # name, GGML type id, rows, cols


def cpu_gemv(ref, synth) -> list:
    """The reference's matmul_quantized (c:2091-2133) on the weight blocks
    and activation the GPU's standalone GEMV lines use (same seeds): median of
    repeated calls, at least 5 and about 0.5 s per shape."""
    import numpy as np

    out = []
    for name, qt, rows, cols in GEMV_SHAPES:
        w = synth.random_blocks(qt, rows, cols, seed=7)
        x = synth.random_x(cols, seed=8)
        y = np.empty(rows, np.float32)
        call = lambda: ref.lib.ref_matmul(qt, w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data)
        call()
        ts, t_end = [], time.perf_counter() + 0.5
        while len(ts) < 5 or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            call()
            ts.append(time.perf_counter() - t0)
        us = float(np.median(ts)) * 1e6
        alg = w.nbytes + 4 * cols + 4 * rows
        out.append({"shape": f"{name} {rows}x{cols}", "us": round(us, 1), "GB/s": round(alg / us / 1e3, 2)})
        del w
    return out


def cpu_leg(path: str, seconds: float, max_tokens: int, kind: str, start: int) -> dict:
    """Runs in a subprocess: greedy decode steps at positions start, start+1,
    ... on the GGUF at path, for about `seconds` (at least one step), by the
    reference engine built with its Makefile's OpenMP line (kind "omp") or
    its basic -O3 line (kind "o3"), or by the oracle ("port").  The steps
    right after opening the model see a zero KV cache below `start`; a
    step's cost (the weight stream and attention over start+1 positions)
    does not depend on what the cache holds.  The "omp" leg then times the
    reference's GEMV at the standalone GEMV shapes."""
    import ctypes

    import numpy as np

    import oracle

    if kind in ("omp", "omp_v4", "o3"):
        ref = oracle.Ref({"omp": oracle.REF_OMP_SO, "omp_v4": oracle.REF_OMP_V4_SO, "o3": oracle.REF_SO}[kind])
        t0 = time.perf_counter()
        if ref.lib.ref_model_open(path.encode(), 0) != 0:
            raise RuntimeError("reference failed to open the model")
        load_s = time.perf_counter() - t0
        tok, n, seed = 1, 0, ctypes.c_ulonglong(42)
        t0 = time.perf_counter()
        while n < max_tokens and (n == 0 or time.perf_counter() - t0 < seconds):
            tok = int(ref.lib.ref_generate_token(tok, start + n, 0.0, 40, 0.9, ctypes.byref(seed)))
            n += 1
        dt = time.perf_counter() - t0
        out = {"tokens": n, "seconds": dt, "load_seconds": load_s}
        if kind.startswith("omp"):
            from llama3pure_amd import synth

            out["gemv"] = cpu_gemv(ref, synth)
        return out
    cr = oracle.CpuRef()
    img = np.fromfile(path, np.uint8)
    t0 = time.perf_counter()
    m = cr.open_model(img.tobytes())
    load_s = time.perf_counter() - t0
    tok, n = 1, 0
    t0 = time.perf_counter()
    while n < max_tokens and (n == 0 or time.perf_counter() - t0 < seconds):
        tok = int(np.argmax(m.forward(tok, start + n)))
        n += 1
    dt = time.perf_counter() - t0
    return {"tokens": n, "seconds": dt, "load_seconds": load_s}


def host_cpu() -> dict:
    """nproc, the CPUs this process may run on, and the CPU model (lscpu)."""
    model = ""
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20)
        for line in r.stdout.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "model": model}


def host_has_avx512() -> bool:
    """Whether the host runs x86-64-v4 code (AVX-512 F, BW, CD, DQ, VL)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags
    except OSError:
        pass
    return False


def run_cpu_leg(path: str, seconds: float, kind: str, threads: int, start: int) -> dict | None:
    env = dict(os.environ, OMP_NUM_THREADS=str(threads))
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-leg", path, "--cpu-seconds", str(seconds),
                        "--cpu-kind", kind, "--cpu-start", str(start)], env=env, capture_output=True, text=True,
                       timeout=900)
    if r.returncode != 0:
        print(r.stderr[-2000:], file=sys.stderr)
        return None
    # the reference prints each decoded token's text to stdout before the result line
    return json.loads(r.stdout[r.stdout.rfind('{"tokens"'):].splitlines()[0])


def cpu_baseline(img, seconds: float, start: int) -> dict | None:
    """The reference on the GPU box's host, decoding at positions >= start of
    the same GGUF: its OpenMP build with the threads this process is given
    (OMP_NUM_THREADS when set, else every CPU of its affinity mask), and its
    basic single-thread -O3 build."""
    import oracle

    cpu = host_cpu()
    use_ref = oracle.have_ref() and os.path.exists(oracle.REF_OMP_SO)
    # the Makefile's -march=native, approximated by the widest ISA level the
    # host runs that a library built elsewhere can target
    v4 = use_ref and os.path.exists(oracle.REF_OMP_V4_SO) and host_has_avx512()
    march = "x86-64-v4" if v4 else "x86-64-v3"
    env_threads = os.environ.get("OMP_NUM_THREADS", "")
    threads = int(env_threads) if env_threads.isdigit() and int(env_threads) > 0 else cpu["affinity"]
    d = "/dev/shm" if os.path.isdir("/dev/shm") else None
    fd, path = tempfile.mkstemp(suffix=".gguf", dir=d)
    try:
        with os.fdopen(fd, "wb") as f:
            img.tofile(f)
        res = run_cpu_leg(path, seconds, ("omp_v4" if v4 else "omp") if use_ref else "port",
                          threads if use_ref else 1, start)
        single = run_cpu_leg(path, seconds, "o3", 1, start) if use_ref else None
    finally:
        os.unlink(path)
    if res is None:
        return None
    where = (f"host: nproc {cpu['nproc']}, {cpu['affinity']} CPUs in this process's affinity mask, "
             f"{cpu['model'] or 'CPU model unknown'}")
    span = lambda r: f"positions {start}..{start + r['tokens'] - 1}"
    if use_ref:
        what = (f"reference C engine, its Makefile's OpenMP line with -march={march} for -march=native "
                f"(-Ofast -fopenmp -march={march}), {threads} threads (OMP_NUM_THREADS={env_threads or 'unset'})")
    else:
        what = "oracle (C restatement of the reference), one thread"
    out = {"value": round(res["tokens"] / res["seconds"], 4), "unit": "tok/s", "cores": threads if use_ref else 1,
           "kind": "reference" if use_ref else "port",
           "sample": f"{what}: {res['tokens']} greedy decode steps at {span(res)} of the same GGUF "
                     f"({res['seconds']:.1f} s; the cache below {start} is zero, which does not change a "
                     f"step's cost: the {img.nbytes / 1e9:.1f} GB weight stream and attention over the "
                     f"positions); {where}",
           "host": cpu}
    if single:
        out["single_thread_O3"] = {
            "value": round(single["tokens"] / single["seconds"], 4), "unit": "tok/s", "cores": 1,
            "sample": f"reference C engine, its Makefile's basic line (gcc -O3), one thread: {single['tokens']} "
                      f"greedy decode steps at {span(single)} ({single['seconds']:.1f} s)"}
    if res.get("gemv"):
        out["gemv"] = res["gemv"]   # matmul_quantized at the standalone GEMV shapes, same blocks and x
    return out


GEMM_TYPES = ("Q8_0", "Q4_K", "Q6_K", "Q5_K", "Q3_K", "Q2_K", "F16", "BF16", "F32",
              "Q4_0", "Q4_1", "Q5_0", "Q5_1", "IQ4_NL")


def gemm_types_only():
    """Batched products (l3p_gemm) of every weight type at 4096 x 4096 and
    1024 rows (Llama-3-8B's output projection over a 1024-position prompt
    pass): random blocks (seed 1) in four copies used in turn, an N(0,1)
    activation (seed 5); three warm calls, then 20 calls between two events on
    the library's stream.  One JSON line per type.  The fp32-MFMA types are
    quoted against the fp32 matrix peak; the Q8_0-activation types run on the
    int8 matrix cores and are quoted against that peak as well."""
    import torch

    import llama3pure_amd as l3p
    from llama3pure_amd import synth

    ctx = l3p.Context(0)
    st = torch.cuda.ExternalStream(ctx.stream)
    rows = cols = 4096
    m = 1024
    x = torch.from_numpy(synth.random_x(cols, seed=5, batch=m)).cuda()
    y = torch.empty(m * rows, dtype=torch.float32, device="cuda")
    flops = 2.0 * rows * cols * m
    for name in GEMM_TYPES:
        qt = getattr(l3p, name)
        w = synth.random_blocks(qt, rows, cols, seed=1)
        wd = [torch.from_numpy(w).cuda() for _ in range(4)]
        torch.cuda.synchronize()
        for i in range(3):
            ctx.gemm(qt, wd[i % 4], rows, cols, x, m, cols, y, rows)
        ctx.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 20
        e0.record(st)
        for i in range(n):
            ctx.gemm(qt, wd[i % 4], rows, cols, x, m, cols, y, rows)
        e1.record(st)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / n
        int8 = name in ("Q4_0", "Q4_1", "Q5_0", "Q5_1", "IQ4_NL")
        tf = flops / us / 1e6
        line = {"type": name, "shape": f"{rows}x{cols} b{m}", "us": round(us, 1), "TFLOP/s": round(tf, 1),
                "matrix_cores": "int8" if int8 else "fp32",
                "frac_of_peak": round(tf / (5000.0 if int8 else 157.3), 4)}
        print(json.dumps(line), flush=True)
        del wd
        torch.cuda.empty_cache()
    ctx.close()


def prefill_types_only(layers: int = 4):
    """A 1024-position prompt (l3p_prefill) through a Llama-3-8B-shape model of
    `layers` layers (dim 4096, FFN 14336, 32 / 8 heads, vocab 1024: the
    projections at full size) for several weight mixes, random blocks;
    the best of three prompts after a warm one, and its GEMM share from the
    per-launch events of one more.  One JSON line per mix."""
    import numpy as np
    import torch

    import llama3pure_amd as l3p
    from llama3pure_amd import synth

    def maker(seed):
        state = [seed]

        def make(qt, rows, cols, std, view):
            state[0] += 1
            view[:] = synth.random_blocks(qt, rows, cols, seed=state[0]).ravel()
            return view

        return make

    mixes = [("Q8_0", l3p.Q8_0, None), ("Q4_0", l3p.Q4_0, None), ("Q5_0", l3p.Q5_0, None),
             ("Q4_K", l3p.Q4_K, None), ("Q4_K, Q6_K attn_v and ffn_down", l3p.Q4_K,
                                        {"attn_v": l3p.Q6_K, "ffn_down": l3p.Q6_K}),
             ("Q6_K", l3p.Q6_K, None)]
    for name, qt, mix in mixes:
        ctx = l3p.Context(0)
        img = synth.synthetic_model(arch="llama", dim=4096, hidden=14336, n_layers=layers, n_heads=32, n_kv=8,
                                    vocab=1024, ctx=2048, qtype=qt, qtypes=mix, make_mat=maker(7))
        mi = ctx.load_gguf(img)
        prompt = np.random.default_rng(5).integers(0, mi.vocab_size, 1024).astype(np.int32)
        ctx.prefill(prompt, 0)
        ctx.synchronize()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            ctx.prefill(prompt, 0)
            ctx.synchronize()
            ts.append(time.perf_counter() - t0)
        ctx.profile(True)
        ctx.prefill(prompt, 0)
        stats = ctx.profile_read()
        ctx.profile(False)
        ms = min(ts) * 1e3
        gemm_ms = sum(v[1] for k, v in stats.items() if " gemm " in k)
        print(json.dumps({"weights": name, "layers": layers, "positions": 1024, "ms": round(ms, 2),
                          "ms_per_layer": round(ms / layers, 3), "gemm_ms": round(gemm_ms, 2)}), flush=True)
        ctx.close()
        del img
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prefill", type=int, default=1024)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-gemv", action="store_true", help="skip the standalone GEMV shapes")
    ap.add_argument("--no-gemma", action="store_true", help="skip the Gemma-2-2B prompt + sampled decode run")
    ap.add_argument("--layers", type=int, default=32,
                    help="layers of the model (32 = Llama-3-8B; fewer only for short counter-collection runs)")
    ap.add_argument("--copy-ceiling", action="store_true",
                    help="only the runtime's device-to-device copy and l3p_stream_read at the GEMV byte sizes "
                         "(an independent check of the streaming-read ceiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only copy 512 MiB device-to-device 5 times (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--gemv-shapes", action="store_true",
                    help="only the standalone GEMV shapes and the streaming-read ceiling at each shape's bytes "
                         "(for a kernel trace or counters)")
    ap.add_argument("--attn-sweep", nargs="?", const="llama3-8b", choices=["llama3-8b", "gemma2b"],
                    help="only run both decode attentions at 65..3001 positions of the named attention shape "
                         "(for a kernel trace)")
    ap.add_argument("--gemm-types", action="store_true",
                    help="only the batched product of every weight type at 4096 x 4096 x 1024 rows")
    ap.add_argument("--prefill-types", action="store_true",
                    help="only a 1024-position prompt through 4 Llama-3-8B-shape layers for several weight mixes")
    ap.add_argument("--cpu-leg", help=argparse.SUPPRESS)
    ap.add_argument("--cpu-kind", default="omp", choices=["omp", "omp_v4", "o3", "port"], help=argparse.SUPPRESS)
    ap.add_argument("--cpu-start", type=int, default=0, help=argparse.SUPPRESS)
    a = ap.parse_args()

    if a.cpu_leg:
        print(json.dumps(cpu_leg(a.cpu_leg, a.cpu_seconds, 64, a.cpu_kind, a.cpu_start)))
        return
    if a.calibrate_copy:
        calibrate_copy()
        return
    if a.copy_ceiling:
        copy_ceiling()
        return
    if a.attn_sweep:
        attn_sweep(a.attn_sweep)
        return
    if a.gemv_shapes:
        gemv_shapes_only()
        return
    if a.gemm_types:
        gemm_types_only()
        return
    if a.prefill_types:
        prefill_types_only()
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X and has no multi-GPU "
              "mode (--gpus must be 1)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import llama3pure_amd as l3p
    from llama3pure_amd import synth

    ctx = l3p.Context(0)
    t0 = time.perf_counter()
    cfg = dict(LLAMA3_8B, n_layers=a.layers)
    img = synth.synthetic_model(qtype=synth.Q8_0, make_mat=synth.gpu_q8_0_maker(ctx, torch, 99), **cfg)
    t_gen = time.perf_counter() - t0
    mi = ctx.load_gguf(img)
    print(f"[bench] model {img.nbytes / 1e9:.2f} GB generated in {t_gen:.1f} s, "
          f"{mi.device_bytes / 1e9:.2f} GB on device", file=sys.stderr, flush=True)

    rng = np.random.default_rng(5)
    prompt = rng.integers(0, mi.vocab_size, a.prefill + 1).astype(np.int32)
    t0 = time.perf_counter()
    ctx.prefill(prompt[:-1], 0)
    t_pre = time.perf_counter() - t0
    print(f"[bench] prefill {a.prefill} positions in {t_pre * 1e3:.1f} ms", file=sys.stderr, flush=True)
    # the same prompt again (it rewrites the same cache rows): timed, then per launch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ctx.prefill(prompt[:-1], 0)
    t_pre = time.perf_counter() - t0
    ctx.profile(True)
    ctx.prefill(prompt[:-1], 0)
    pstats = ctx.profile_read()
    ctx.profile(False)
    prefill = prefill_summary(a.prefill, t_pre, pstats)
    print(f"[bench] prefill: {json.dumps(prefill)}", file=sys.stderr, flush=True)

    def run(n, tok, pos):
        for _ in range(n):
            tok, _ = ctx.decode(tok, pos, temperature=0.0)
            pos += 1
        return tok, pos

    def run_queued(n, tok, pos):
        toks = ctx.generate_greedy(tok, pos, n)
        assert len(toks) == n, (len(toks), n)
        return toks[-1], pos + n

    assert a.prefill + a.warmup + 3 * a.steps <= mi.seq_len, "steps exceed the 2048-position context"
    tok, pos = run(a.warmup, int(prompt[-1]), a.prefill)
    ctx.synchronize()
    torch.cuda.synchronize()
    # the timed steps: the reference's greedy loop as one l3p_generate_greedy
    # call (each step's token read back while the next step runs)
    t0 = time.perf_counter()
    tok, pos = run_queued(a.steps, tok, pos)
    ctx.synchronize()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    tps = a.steps / dt
    print(f"[bench] {a.steps} decode steps in {dt * 1e3:.1f} ms: {tps:.1f} tok/s", file=sys.stderr, flush=True)
    # the same number of steps as one l3p_decode call per token from Python
    t0 = time.perf_counter()
    tok, pos = run(a.steps, tok, pos)
    ctx.synchronize()
    torch.cuda.synchronize()
    dt_call = time.perf_counter() - t0
    print(f"[bench] {a.steps} l3p_decode calls in {dt_call * 1e3:.1f} ms: {a.steps / dt_call:.1f} tok/s",
          file=sys.stderr, flush=True)

    # second pass with per-kernel dispatch events: the roofline of the dominant GEMV class
    ctx.profile(True)
    tok, pos = run(a.steps, tok, pos)
    stats = ctx.profile_read()
    ctx.profile(False)
    name, (launches, ms, bpl) = max(stats.items(), key=lambda kv: kv[1][1])
    avg_us = ms * 1e3 / launches
    achieved = bpl / (avg_us * 1e-6) / 1e9
    kernels = {k: {"launches": v[0], "avg_us": round(v[1] * 1e3 / v[0], 2),
                   "GB/s": round(v[2] / (v[1] * 1e-3 / v[0]) / 1e9, 1)} for k, v in stats.items()}
    print(f"[bench] GEMV classes: {json.dumps(kernels)}", file=sys.stderr, flush=True)

    ceiling = {"read_2GiB": round(read_ceiling(ctx, torch, 2 << 30), 1),
               "read_same_bytes": round(read_ceiling(ctx, torch, int(bpl)), 1)}
    print(f"[bench] streaming-read ceiling (GB/s): {json.dumps(ceiling)}", file=sys.stderr, flush=True)
    gemv = None if a.no_gemv else time_gemv_shapes(ctx, torch, l3p, synth)
    if gemv:
        print(f"[bench] standalone GEMV: {json.dumps(gemv)}", file=sys.stderr, flush=True)

    base = None if a.no_cpu else cpu_baseline(img, a.cpu_seconds, a.prefill)
    del img
    ctx.close()
    gemma = None if a.no_gemma else gemma_prompt_decode(np, torch, l3p, synth)
    if gemma:
        print(f"[bench] gemma-2-2b: {json.dumps(gemma)}", file=sys.stderr, flush=True)

    line = {
        "metric": "quant GEMV HBM GB/s (% of peak); decode tok/s Llama-3-8B-arch Q8_0, 1 GPU",
        "value": round(tps, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dt * 1e3 / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights (int8 quants, fp16 block scales); fp32 activations and accumulation",
        "data": "synthetic: random-init weights N(0,0.02) quantized to Q8_0, uniform random token ids",
        "config": {"workload": "greedy decode, Llama-3-8B architecture, all matrices Q8_0, KV prefilled to "
                               f"{a.prefill} of 2048", "layers": a.layers, "dim": 4096, "heads": 32, "kv_heads": 8,
                   "ffn": 14336, "vocab": 128256, "start_pos": a.prefill, "parallelism": "single GPU",
                   "decode_call": "l3p_generate_greedy (steps queued two ahead of the host's token reads)"},
        "per_call_decode": {"call": "l3p_decode once per token from Python (synchronous)",
                            "tok_s": round(a.steps / dt_call, 3), "ms_per_step": round(dt_call * 1e3 / a.steps, 4)},
        "roofline": {"bound": "hbm", "kernel": name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(name),
                     "bytes_per_launch": int(bpl), "avg_launch_us": round(avg_us, 2), "launches": launches,
                     "read_ceiling_GBps": ceiling,
                     "frac_of_read_ceiling": round(achieved / ceiling["read_same_bytes"], 4)},
        "gemv_classes": kernels,
        "prefill": prefill,
        "gemv": gemv,
        "gemma_2b_prompt_decode": gemma,
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
