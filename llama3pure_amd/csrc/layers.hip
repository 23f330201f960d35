// layers.hip — the fused per-layer kernels of the decode path (gfx950):
// RMSNorm (+ activation quantization), QK-norm + RoPE + Q8_0 KV write,
// split-position GQA attention over the Q8_0 KV cache, logit soft-cap and the
// sampler.  Arithmetic follows llama3pure-c-engine.c (cited per kernel); the
// library is built with -ffp-contract=off so elementwise expressions round
// exactly as the reference's scalar C does.
#include "model.h"

#include <hip/hip_fp16.h>

namespace {

constexpr int kTC = 64;   // positions per attention chunk (one per lane)

__device__ __forceinline__ float h2f(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
}
__device__ __forceinline__ float h2f_exact(uint32_t h) {
    h &= 0xffffu;
    if (((h >> 10) & 31u) == 31u)
        return __uint_as_float(((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13));
    return h2f(h);
}
__device__ __forceinline__ uint32_t f2h_trunc(float f) {   // c:585-599
    uint32_t b = __float_as_uint(f);
    uint32_t sign = (b >> 16) & 0x8000u;
    int e = (int)((b >> 23) & 0xffu) - 112;
    uint32_t m = (b >> 13) & 0x3ffu;
    if (e <= 0) {
        if (e < -10) return sign;
        return sign | ((m | 0x400u) >> (1 - e));
    }
    if (e >= 31) return sign | 0x7c00u;
    return sign | ((uint32_t)e << 10) | m;
}
__device__ __forceinline__ uint32_t shr64(uint32_t lo, uint32_t hi, uint32_t sh) {
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> sh);
}
__device__ __forceinline__ float ref_fast_tanhf(float x) {   // c:3089-3095
    if (x < -4.0f) return -1.0f;
    if (x > 4.0f) return 1.0f;
    float x2 = x * x;
    return (x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2)))) /
           (135135.0f + x2 * (62370.0f + x2 * (3150.0f + 28.0f * x2)));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over the workgroup (any size that is a multiple of 64, <= 1024).
__device__ float block_sum(float v, float* sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; ++i) s += sh[i];
    return s;
}

// Q8_0 quantization of 32 values (quantize_row_q8_0, c:1508-1528): truncated
// fp16 scale d = amax/127, q = roundf(x * (127/amax)).
struct QBlock {
    uint32_t dh;
    int8_t q[32];
    int sum;
};
__device__ __forceinline__ void quantize32(const float* v, QBlock& o) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        float a = v[j] < 0 ? -v[j] : v[j];
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;
    o.dh = f2h_trunc(d);
    int s = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        int qi = (int)roundf(v[j] * id);
        qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
        o.q[j] = (int8_t)qi;
        s += qi;
    }
    o.sum = s;
}
__device__ __forceinline__ void store_block34(uint8_t* dst, const QBlock& b) {
    dst[0] = (uint8_t)(b.dh & 0xff);
    dst[1] = (uint8_t)(b.dh >> 8);
#pragma unroll
    for (int j = 0; j < 32; ++j) dst[2 + j] = (uint8_t)b.q[j];
}

// ---------------------------------------------------------------------------
// RMSNorm (c:3117-3129), optional fused embedding scale (Gemma first layer,
// c:3132-3148) and optional Q8_0 quantization of the output for the integer
// GEMV path.  One workgroup.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024) rmsnorm_kernel(const float* __restrict__ xin, float* xscale, float scale,
                                                       const float* __restrict__ w, int n, float inv_n, float eps,
                                                       float* out, XQ8 xq, int do_q) {
    __shared__ float sh[16];
    const int t = threadIdx.x, nt = blockDim.x;
    float ss = 0.0f;
    for (int j = t; j < n; j += nt) {
        float v = xin[j];
        if (xscale) {
            v = v * scale;
            xscale[j] = v;
        }
        ss += v * v;
    }
    ss = block_sum(ss, sh);
    const float r = 1.0f / sqrtf(ss * inv_n + eps);
    const float* xs = xscale ? xscale : xin;
    __syncthreads();
    for (int b = t; b < n / 32; b += nt) {
        float o[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) o[j] = w[32 * b + j] * (r * xs[32 * b + j]);
#pragma unroll
        for (int j = 0; j < 32; ++j) out[32 * b + j] = o[j];
        if (do_q) {
            QBlock qb;
            quantize32(o, qb);
#pragma unroll
            for (int j = 0; j < 32; ++j) xq.qs[32 * b + j] = qb.q[j];
            xq.d[b] = h2f_exact(qb.dh);
            xq.sum[b] = qb.sum;
        }
    }
}

// x += rmsnorm(y) (Gemma post-attention / post-FFN norm then residual,
// c:3364-3371, c:3411-3417).
__global__ void __launch_bounds__(1024) rmsnorm_add_kernel(const float* __restrict__ y, const float* __restrict__ w,
                                                           int n, float inv_n, float eps, float* x) {
    __shared__ float sh[16];
    const int t = threadIdx.x, nt = blockDim.x;
    float ss = 0.0f;
    for (int j = t; j < n; j += nt) ss += y[j] * y[j];
    ss = block_sum(ss, sh);
    const float r = 1.0f / sqrtf(ss * inv_n + eps);
    for (int j = t; j < n; j += nt) x[j] += w[j] * (r * y[j]);
}

// ---------------------------------------------------------------------------
// Per head: Gemma QK-norm (c:3151-3165), RoPE with attn_scale fused into Q
// (c:3240-3296), Q8_0 quantization of K and V into the cache at pos
// (c:3301-3308) and of Q for the integer scores (c:3311-3312).
// Workgroup = one wave; blocks [0, n_heads) are query heads, then KV heads.
// ---------------------------------------------------------------------------
struct RopeArgs {
    float *q, *k;
    const float* v;
    const float *q_norm, *k_norm;
    const float *cos, *sin;      // rows for this position
    uint8_t *kc, *vc;            // cache slots [n_kv][seq][hq8] at this position (layer base + pos*hq8)
    size_t head_seq;
    int8_t* qq;                  // [n_heads][hs]
    float* qd;                   // [n_heads][hs/32]
    int n_heads, hs, neox;
    float attn_scale, eps, inv_hs;
};

__global__ void __launch_bounds__(64) rope_kv_kernel(RopeArgs a) {
    __shared__ float hv[256 + 8];
    const int lane = threadIdx.x;
    const bool isq = (int)blockIdx.x < a.n_heads;
    const int head = isq ? blockIdx.x : blockIdx.x - a.n_heads;
    const int hs = a.hs, half = hs / 2;
    float* src = (isq ? a.q : a.k) + (size_t)head * hs;

    // QK-norm (per-head rmsnorm) when weights are present
    const float* nw = isq ? a.q_norm : a.k_norm;
    for (int j = lane; j < hs; j += 64) hv[j] = src[j];
    __syncthreads();
    if (nw) {
        float ss = 0.0f;
        for (int j = lane; j < hs; j += 64) ss += hv[j] * hv[j];
        ss = wave_sum(ss);
        const float r = 1.0f / sqrtf(ss * a.inv_hs + a.eps);
        __syncthreads();
        for (int j = lane; j < hs; j += 64) hv[j] = nw[j] * (r * hv[j]);
        __syncthreads();
    }
    // RoPE
    for (int p = lane; p < half; p += 64) {
        const float c = a.cos[p], s = a.sin[p];
        const int i0 = a.neox ? p : 2 * p;
        const int i1 = a.neox ? p + half : 2 * p + 1;
        const float v0 = hv[i0], v1 = hv[i1];
        if (isq) {
            hv[i0] = (v0 * c - v1 * s) * a.attn_scale;
            hv[i1] = (v0 * s + v1 * c) * a.attn_scale;
        } else {
            hv[i0] = v0 * c - v1 * s;
            hv[i1] = v0 * s + v1 * c;
        }
    }
    __syncthreads();
    for (int j = lane; j < hs; j += 64) src[j] = hv[j];
    const int nb = hs / 32;
    if (lane < nb) {
        QBlock qb;
        quantize32(hv + 32 * lane, qb);
        if (isq) {
            int8_t* dq = a.qq + (size_t)head * hs + 32 * lane;
#pragma unroll
            for (int j = 0; j < 32; ++j) dq[j] = qb.q[j];
            a.qd[head * nb + lane] = h2f_exact(qb.dh);
        } else {
            store_block34(a.kc + (size_t)head * a.head_seq + 34 * lane, qb);
        }
    } else if (!isq && lane >= 32 && lane < 32 + nb) {
        const int b = lane - 32;
        float vv[32];
        const float* vs = a.v + (size_t)head * hs + 32 * b;
#pragma unroll
        for (int j = 0; j < 32; ++j) vv[j] = vs[j];
        QBlock qb;
        quantize32(vv, qb);
        store_block34(a.vc + (size_t)head * a.head_seq + 34 * b, qb);
    }
}

// ---------------------------------------------------------------------------
// Attention over the Q8_0 cache (c:3314-3359), split over chunks of 64
// positions.  Kernel 1: integer scores per position, bit-exact with
// dot_q8_0_q8_0_cache (c:1574-1597); the last chunk of each KV group to
// finish runs the softmax (c:3167-3186) for the group's query heads and
// stores the normalized weights.  Kernel 2: weighted V accumulation
// (accum_q8_0_cache, c:1600-1622, weights |w| < 1e-8 skipped) per chunk; the
// last chunk of a group sums the chunk partials in chunk order.
// Workgroup = kv_mul waves (one per query head of the group) x one chunk.
// ---------------------------------------------------------------------------
struct AttnKArgs {
    const int8_t* qq;
    const float* qd;
    const uint8_t* kc;
    const uint8_t* vc;
    float* att;
    float* part_acc;
    unsigned* counters;
    float* out;
    size_t head_seq;
    int n_heads, kv_mul, hs, hq8, seq, t0, na, n_chunks;
};

__global__ void __launch_bounds__(1024) attn_scores_kernel(AttnKArgs a) {
    __shared__ unsigned last;
    const int g = blockIdx.x, c = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = g * a.kv_mul + w;
    const int nb = a.hs / 32;
    const int i = c * kTC + lane;         // position index relative to t0
    if (i < a.na) {
        const int t = a.t0 + i;
        const uint8_t* row = a.kc + (size_t)g * a.head_seq + (size_t)t * a.hq8;
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(row);   // rows are 4-byte aligned
        const int8_t* qh = a.qq + (size_t)h * a.hs;
        float sum = 0.0f;
        for (int b = 0; b < nb; ++b) {
            const uint32_t off = 34u * b;
            const uint32_t E = off >> 2, sh = (off & 2u) ? 32u : 16u;
            uint32_t dw[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) dw[k] = rw[E + k];
            const float db = h2f(dw[0] >> ((off & 2u) ? 16u : 0u));
            const int4* qp = reinterpret_cast<const int4*>(qh + 32 * b);
            const int4 qa = qp[0], qb4 = qp[1];
            const int qv[8] = {qa.x, qa.y, qa.z, qa.w, qb4.x, qb4.y, qb4.z, qb4.w};
            int isum = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) isum = __builtin_amdgcn_sdot4(qv[k], (int)shr64(dw[k], dw[k + 1], sh), isum, false);
            const float da = a.qd[h * nb + b];
            sum += da * db * (float)isum;
        }
        a.att[(size_t)h * a.seq + i] = sum;
    }
    // the last chunk of this KV group runs the softmax for the group's heads
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(&a.counters[g], 1u) == (unsigned)(a.n_chunks - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    float* att = a.att + (size_t)h * a.seq;
    float m = -INFINITY;
    for (int j = lane; j < a.na; j += 64) m = fmaxf(m, att[j]);
    m = wave_max(m);
    float s = 0.0f;
    for (int j = lane; j < a.na; j += 64) {
        const float e = expf(att[j] - m);
        att[j] = e;
        s += e;
    }
    s = wave_sum(s);
    const float inv = 1.0f / s;
    for (int j = lane; j < a.na; j += 64) att[j] *= inv;
    __syncthreads();
    if (threadIdx.x == 0) a.counters[g] = 0;
}

__global__ void __launch_bounds__(1024) attn_values_kernel(AttnKArgs a) {
    __shared__ unsigned last;
    const int g = blockIdx.x, c = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = g * a.kv_mul + w;
    const int per = a.hs / 64;                 // outputs per lane (2 or 4)
    const int i0 = lane * per;                 // first output element of this lane
    const int b = i0 >> 5;                     // its 32-block
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* att = a.att + (size_t)h * a.seq;
    const uint8_t* vbase = a.vc + (size_t)g * a.head_seq + 34 * b;
    const int jbeg = c * kTC, jend = min(a.na, jbeg + kTC);
    for (int j = jbeg; j < jend; ++j) {
        const float wt = att[j];
        if (wt > -1e-8f && wt < 1e-8f) continue;
        const uint8_t* blk = vbase + (size_t)(a.t0 + j) * a.hq8;
        const float scale = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8)) * wt;
        const int8_t* qs = reinterpret_cast<const int8_t*>(blk + 2 + (i0 & 31));
        for (int e = 0; e < per; ++e) acc[e] += (float)qs[e] * scale;
    }
    float* out = a.out + (size_t)h * a.hs + i0;
    if (a.n_chunks == 1) {
        for (int e = 0; e < per; ++e) out[e] = acc[e];
        return;
    }
    float* pa = a.part_acc + ((size_t)h * a.n_chunks + c) * a.hs + i0;
    for (int e = 0; e < per; ++e) pa[e] = acc[e];
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(&a.counters[g], 1u) == (unsigned)(a.n_chunks - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    float tot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int cc = 0; cc < a.n_chunks; ++cc) {
        const float* p = a.part_acc + ((size_t)h * a.n_chunks + cc) * a.hs + i0;
        for (int e = 0; e < per; ++e) tot[e] += p[e];
    }
    for (int e = 0; e < per; ++e) out[e] = tot[e];
    __syncthreads();
    if (threadIdx.x == 0) a.counters[g] = 0;
}

// Final logit soft-cap (Gemma, c:3425-3433).
__global__ void softcap_kernel(float* l, int n, float cap) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) l[i] = cap * ref_fast_tanhf(l[i] / cap);
}

// ---------------------------------------------------------------------------
// Sampler.  argmax (c:4278-4288): the first index of the maximum.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

__global__ void __launch_bounds__(1024) argmax_partial_kernel(const float* __restrict__ l, int n, float* cv, int* ci) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        if (better(l[i], i, bv, bi)) { bv = l[i]; bi = i; }
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x >> 6); ++k)
            if (better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
        cv[blockIdx.x] = bv;
        ci[blockIdx.x] = bi;
    }
}

__global__ void argmax_final_kernel(const float* cv, const int* ci, int nc, int* out) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int k = threadIdx.x; k < nc; k += 64)
        if (better(cv[k], ci[k], bv, bi)) { bv = cv[k]; bi = ci[k]; }
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (threadIdx.x == 0) *out = bi == 0x7fffffff ? 0 : bi;
}

// Top-k / temperature / top-p (c:4803-4907).  Stage 1 sorts chunks of 1024
// logits in LDS (value descending, index ascending) and keeps each chunk's
// best k; stage 2 sorts the candidates and runs the reference's sampling
// arithmetic on the best k in descending order.
constexpr int kChunk = 1024;
constexpr int kMaxK = 128;

__device__ void bitonic_sort_desc(float* v, int* id, int n) {   // n power of two
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int i = threadIdx.x; i < n / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const bool swap = desc ? better(v[hi], id[hi], v[lo], id[lo]) : better(v[lo], id[lo], v[hi], id[hi]);
                if (swap) {
                    float tv = v[lo]; v[lo] = v[hi]; v[hi] = tv;
                    int ti = id[lo]; id[lo] = id[hi]; id[hi] = ti;
                }
            }
        }
    }
    __syncthreads();
}

__global__ void __launch_bounds__(1024) topk_stage1_kernel(const float* __restrict__ l, int n, int k, float* cv, int* ci) {
    __shared__ float v[kChunk];
    __shared__ int id[kChunk];
    const int base = blockIdx.x * kChunk;
    for (int i = threadIdx.x; i < kChunk; i += blockDim.x) {
        const int gi = base + i;
        v[i] = gi < n ? l[gi] : -INFINITY;
        id[i] = gi < n ? gi : 0x7fffffff;
    }
    bitonic_sort_desc(v, id, kChunk);
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        cv[blockIdx.x * k + i] = v[i];
        ci[blockIdx.x * k + i] = id[i];
    }
}

__global__ void __launch_bounds__(1024) topk_stage2_kernel(const float* cv, const int* ci, int nc, int np2, int k,
                                                           float temperature, float top_p, float r, int* out) {
    extern __shared__ float smem[];
    float* v = smem;
    int* id = reinterpret_cast<int*>(smem + np2);
    for (int i = threadIdx.x; i < np2; i += blockDim.x) {
        v[i] = i < nc ? cv[i] : -INFINITY;
        id[i] = i < nc ? ci[i] : 0x7fffffff;
    }
    bitonic_sort_desc(v, id, np2);
    if (threadIdx.x != 0) return;
    // the reference's arithmetic on the k best, in descending order
    const float inv_t = 1.0f / temperature;
    const float max_vt = v[0] * inv_t;
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) {
        const float e = expf(v[i] * inv_t - max_vt);
        v[i] = e;
        sum += e;
    }
    int keep = k;
    if (top_p < 1.0f) {
        float cum = 0.0f;
        const float thr = top_p * sum;
        for (int i = 0; i < k; ++i) {
            cum += v[i];
            if (cum >= thr) { keep = i + 1; break; }
        }
        sum = 0.0f;
        for (int i = 0; i < keep; ++i) sum += v[i];
    }
    const float rr = r * sum;
    float cdf = 0.0f;
    int s = keep - 1;
    for (int i = 0; i < keep; ++i) {
        cdf += v[i];
        if (rr < cdf) { s = i; break; }
    }
    *out = id[s];
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
void launch_embed(const Mat& emb, int token, float* x, hipStream_t s) {
    launch_dequant(emb.type, emb.w + (size_t)token * emb.rb, emb.cols, x, s);
}

void launch_rmsnorm(const float* xin, float* xscale, float scale, const float* w, int n, float inv_n, float eps,
                    float* out, const XQ8* xq, hipStream_t s) {
    XQ8 q = xq ? *xq : XQ8{};
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, xin, xscale, scale, w, n, inv_n, eps, out, q,
                       xq ? 1 : 0);
    L3P_HIP(hipGetLastError());
}

void launch_rmsnorm_add(const float* y, const float* w, int n, float inv_n, float eps, float* x, hipStream_t s) {
    hipLaunchKernelGGL(rmsnorm_add_kernel, dim3(1), dim3(1024), 0, s, y, w, n, inv_n, eps, x);
    L3P_HIP(hipGetLastError());
}

void launch_rope_kv(const Model& m, int l, int pos, hipStream_t s) {
    const Layer& L = m.layers[l];
    const bool swa = m.swa_pattern > 0 && (l % m.swa_pattern < m.swa_pattern - 1);   // c:3247
    const bool use_swa_tables = m.is_gemma && swa;
    const int half = m.hs / 2;
    RopeArgs a;
    a.q = m.q;
    a.k = m.k;
    a.v = m.v;
    a.q_norm = m.is_gemma ? L.q_norm : nullptr;
    a.k_norm = m.is_gemma ? L.k_norm : nullptr;
    a.cos = (use_swa_tables ? m.cos_s : m.cos_d) + (size_t)pos * half;
    a.sin = (use_swa_tables ? m.sin_s : m.sin_d) + (size_t)pos * half;
    const size_t loff = (size_t)l * m.layer_kv + (size_t)pos * m.hq8;
    a.kc = m.kc + loff;
    a.vc = m.vc + loff;
    a.head_seq = m.head_seq;
    a.qq = m.qq;
    a.qd = m.qd;
    a.n_heads = m.n_heads;
    a.hs = m.hs;
    a.neox = m.is_gemma;
    a.attn_scale = m.attn_scale;
    a.eps = m.eps > 0 ? m.eps : 1e-5f;
    a.inv_hs = m.inv_hs;
    hipLaunchKernelGGL(rope_kv_kernel, dim3(m.n_heads + m.n_kv), dim3(64), 0, s, a);
    L3P_HIP(hipGetLastError());
}

void launch_attention(const AttnArgs& x, hipStream_t s) {
    AttnKArgs a;
    a.qq = x.qq;
    a.qd = x.qd;
    a.kc = x.kc;
    a.vc = x.vc;
    a.att = x.att;
    a.part_acc = x.part_acc;
    a.counters = x.counters;
    a.out = x.out;
    a.head_seq = x.head_seq;
    a.n_heads = x.n_heads;
    a.kv_mul = x.kv_mul;
    a.hs = x.hs;
    a.hq8 = x.hq8;
    a.seq = x.seq;
    a.t0 = x.t0;
    a.na = x.na;
    a.n_chunks = (x.na + kTC - 1) / kTC;
    const dim3 grid(x.n_heads / x.kv_mul, a.n_chunks), block(64 * x.kv_mul);
    hipLaunchKernelGGL(attn_scores_kernel, grid, block, 0, s, a);
    L3P_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_values_kernel, grid, block, 0, s, a);
    L3P_HIP(hipGetLastError());
}

void launch_softcap(float* l, int n, float cap, hipStream_t s) {
    hipLaunchKernelGGL(softcap_kernel, dim3((n + 255) / 256), dim3(256), 0, s, l, n, cap);
    L3P_HIP(hipGetLastError());
}

int sample_num_blocks(int n) { return (n + kChunk - 1) / kChunk; }
int sample_candidates_per_block() { return kMaxK; }

void launch_argmax(const float* l, int n, int* out, hipStream_t s, float* cv, int* ci) {
    const int nb = 256;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(nb), dim3(1024), 0, s, l, n, cv, ci);
    L3P_HIP(hipGetLastError());
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, s, cv, ci, nb, out);
    L3P_HIP(hipGetLastError());
}

void launch_sample_topk(const float* l, int n, float temperature, int k, float top_p, float r, float* cv, int* ci,
                        int* out, hipStream_t s) {
    L3P_REQUIRE(k >= 1 && k <= kMaxK, L3P_E_UNSUPPORTED, "sampler: top_k=%d outside [1, %d]", k, kMaxK);
    const int nb = sample_num_blocks(n);
    hipLaunchKernelGGL(topk_stage1_kernel, dim3(nb), dim3(1024), 0, s, l, n, k, cv, ci);
    L3P_HIP(hipGetLastError());
    const int nc = nb * k;
    int np2 = 1;
    while (np2 < nc) np2 <<= 1;
    const size_t lds = (size_t)np2 * 8;
    L3P_REQUIRE(lds <= 160 * 1024, L3P_E_UNSUPPORTED, "sampler: %d candidates exceed LDS", nc);
    if (lds > 65536)
        L3P_HIP(hipFuncSetAttribute((const void*)topk_stage2_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(topk_stage2_kernel, dim3(1), dim3(1024), lds, s, cv, ci, nc, np2, k, temperature, top_p, r, out);
    L3P_HIP(hipGetLastError());
}
