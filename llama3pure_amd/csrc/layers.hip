// layers.hip — the fused per-layer kernels of the decode path (gfx950):
// RMSNorm (+ activation quantization), QK-norm + RoPE + Q8_0 KV write,
// split-position GQA attention over the Q8_0 KV cache, logit soft-cap and the
// sampler.  Arithmetic follows llama3pure-c-engine.c (cited per kernel); the
// library is built with -ffp-contract=off so elementwise expressions round
// exactly as the reference's scalar C does.
#include "device_common.h"
#include "model.h"

namespace {

constexpr int kTC = 64;   // positions per attention chunk (one per lane)
typedef __attribute__((address_space(3))) void lds_void;

using namespace l3pd;

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

__device__ __forceinline__ void store_block34(uint8_t* dst, const QBlock& b) {
    dst[0] = (uint8_t)(b.dh & 0xff);
    dst[1] = (uint8_t)(b.dh >> 8);
#pragma unroll
    for (int j = 0; j < 32; ++j) dst[2 + j] = (uint8_t)b.q[j];
}

// ---------------------------------------------------------------------------
// RMSNorm (c:3117-3129), optional fused embedding scale (Gemma first layer,
// c:3132-3148), and the output also written in the form the next GEMV
// consumes (form 1: Q8_0 for Q4_0 weights; form 2: digits for Q8_0 weights).
// One workgroup.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024) rmsnorm_kernel(const float* __restrict__ xin, float* xscale, float scale,
                                                       const float* __restrict__ w, int n, float inv_n, float eps,
                                                       float* out, XQ8 xq, XDig xd, int form) {
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
        if (form == 1) {
            QBlock qb;
            quantize32(o, qb);
            int4* dq = reinterpret_cast<int4*>(xq.qs + 32 * b);
            const int* qi = reinterpret_cast<const int*>(qb.q);
            dq[0] = make_int4(qi[0], qi[1], qi[2], qi[3]);
            dq[1] = make_int4(qi[4], qi[5], qi[6], qi[7]);
            xq.d[b] = h2f_exact(qb.dh);
            xq.sum[b] = qb.sum;
        } else if (form == 2) {
            int8_t dg[4][32];
            const float sc = digits32(o, dg);
            int4* dd = reinterpret_cast<int4*>(xd.dg + 128 * b);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int* p = reinterpret_cast<const int*>(dg[k]);
                dd[2 * k] = make_int4(p[0], p[1], p[2], p[3]);
                dd[2 * k + 1] = make_int4(p[4], p[5], p[6], p[7]);
            }
            xd.s[b] = sc;
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
// positions; workgroup = kv_mul waves (one per query head of a KV group) x
// one chunk.
//   attn_scores_kernel: lane = position; the score is the reference's
//     dot_q8_0_q8_0_cache (c:1574-1597): exact integer block dots, fp32 sum
//     over blocks in block order, so scores are bit-exact.
//     Each chunk also leaves its maximum and its sum of expf(s - chunk max).
//   attn_values_kernel: every workgroup combines the chunk maxima and sums
//     into the head's softmax max M and sum S (softmax, c:3167-3186; the same
//     order in every workgroup), forms its chunk's weights
//     w = expf(s - M) * (1/S), and
//     accum_q8_0_cache (c:1600-1622: out += q * (d * w), |w| < 1e-8 skipped)
//     over its chunk's V rows staged in LDS, into a per-chunk partial;
//   attn_combine_kernel: adds the chunk partials in chunk order.
// ---------------------------------------------------------------------------
struct AttnKArgs {
    const int8_t* qq;
    const float* qd;
    const uint8_t* kc;      // allocation base of the K cache (256-byte aligned)
    const uint8_t* vc;      // allocation base of the V cache
    size_t layer_off;       // byte offset of this layer in both caches
    float* att;
    float* part_acc;
    float* part_ms;         // [n_heads][2][n_chunks]: chunk max, chunk sum of expf(s - max)
    float* out;
    size_t head_seq;
    int n_heads, kv_mul, hs, hq8, seq, t0, na, n_chunks;
};

__global__ void __launch_bounds__(1024) attn_scores_kernel(AttnKArgs a) {
    const int g = blockIdx.x, c = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = g * a.kv_mul + w;
    const int nb = a.hs / 32;
    const int i = c * kTC + lane;         // position index relative to t0
    if (i < a.na) {
    const int t = a.t0 + i;
    // absolute byte offset of the K row from the (256-byte aligned) cache base
    const size_t rowoff = a.layer_off + (size_t)g * a.head_seq + (size_t)t * a.hq8;
    const uint32_t* cw = reinterpret_cast<const uint32_t*>(a.kc);
    const int8_t* qh = a.qq + (size_t)h * a.hs;
    float sum = 0.0f;
#pragma unroll 8
    for (int b = 0; b < nb; ++b) {
        const size_t off = rowoff + 34u * b;
        const size_t E = off >> 2;
        const uint32_t sh = (off & 2u) ? 32u : 16u;
        uint32_t dw[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) dw[k] = cw[E + k];
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
    // chunk statistics for the softmax
    const float v = i < a.na ? a.att[(size_t)h * a.seq + i] : -INFINITY;
    const float cm = wave_max(v);
    const float cs = wave_sum(i < a.na ? expf(v - cm) : 0.0f);
    if (lane == 0) {
        a.part_ms[((size_t)h * 2) * a.n_chunks + c] = cm;
        a.part_ms[((size_t)h * 2 + 1) * a.n_chunks + c] = cs;
    }
}

__global__ void __launch_bounds__(1024) attn_values_kernel(AttnKArgs a) {
    extern __shared__ __align__(16) float smem[];
    const int g = blockIdx.x, c = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nt = blockDim.x;
    const int h = g * a.kv_mul + w;
    const float* att = a.att + (size_t)h * a.seq;

    // V rows of this chunk -> LDS, copied HBM -> LDS by global_load_lds_dword
    // (64 dwords per instruction) from the 4-byte aligned start, all issued
    // before anything waits
    const int jbeg = c * kTC, jend = min(a.na, jbeg + kTC);
    const size_t start = a.layer_off + (size_t)g * a.head_seq + (size_t)(a.t0 + jbeg) * a.hq8;
    const size_t end = start + (size_t)(jend - jbeg) * a.hq8;
    const size_t s4 = start & ~(size_t)3;
    const int nd = (int)((end - s4 + 3) >> 2);
    float* wts = smem;                                                      // [kv_mul][8][kTC]
    uint32_t* vb = reinterpret_cast<uint32_t*>(smem + a.kv_mul * 8 * kTC);  // chunk V rows
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.vc) + (s4 >> 2);
    const int nw = nt >> 6;
    for (int i = w; i * 64 < nd; i += nw) {
        if (i * 64 + lane < nd)
            __builtin_amdgcn_global_load_lds(src + i * 64 + lane, (lds_void*)(vb + i * 64), 4, 0, 0);
    }

    // softmax max and sum of head h (c:3167-3186) from the chunk statistics
    const float* pm = a.part_ms + ((size_t)h * 2) * a.n_chunks;
    const float* ps = pm + a.n_chunks;
    float m = -INFINITY;
    for (int cc = lane; cc < a.n_chunks; cc += 64) m = fmaxf(m, pm[cc]);
    m = wave_max(m);
    float ssum = 0.0f;
    for (int cc = lane; cc < a.n_chunks; cc += 64) ssum += ps[cc] * expf(pm[cc] - m);
    ssum = wave_sum(ssum);
    const float inv = 1.0f / ssum;
    const float wt = jbeg + lane < jend ? expf(att[jbeg + lane] - m) * inv : 0.0f;
    __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0): this wave's V copies have landed
    __syncthreads();

    // f[b][j] = d(row j, block b) * w_j, or 0 where the reference skips
    // position j (|w| < 1e-8); then out[i] += q[j][i] * f[b(i)][j]
    // (accum_q8_0_cache, c:1600-1622: scale = d * w, out += q * scale)
    const int nbk = a.hs / 32;
    const uint8_t* rows = reinterpret_cast<const uint8_t*>(vb) + (start - s4);
    float* f = wts + (size_t)w * 8 * kTC;     // [8][kTC] for this head
    if (jbeg + lane < jend) {
        const bool skip = wt > -1e-8f && wt < 1e-8f;
        for (int bb = 0; bb < nbk; ++bb) {
            const uint8_t* sc = rows + (size_t)lane * a.hq8 + 34 * bb;
            const float d = h2f((uint32_t)sc[0] | ((uint32_t)sc[1] << 8));
            f[bb * kTC + lane] = skip ? 0.0f : d * wt;
        }
    }
    __syncthreads();
    const int per = (a.hs + 63) / 64;          // outputs per lane (1, 2 or 4)
    const int i0 = lane * per;                 // first output element of this lane
    const bool act = i0 < a.hs;
    const int b = act ? i0 >> 5 : 0;           // its 32-block
    const uint8_t* qrow = rows + 34 * b + 2 + (i0 & 31);
    const float* fb = f + b * kTC;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int cnt = jend - jbeg;
    if (act) {
        if (per == 2) {
#pragma unroll 8
            for (int j = 0; j < cnt; ++j) {
                const uint32_t q = *reinterpret_cast<const uint16_t*>(qrow + (size_t)j * a.hq8);
                const float fj = fb[j];
                acc[0] += (float)(int8_t)(q & 0xffu) * fj;
                acc[1] += (float)(int8_t)(q >> 8) * fj;
            }
        } else {
#pragma unroll 4
            for (int j = 0; j < cnt; ++j) {
                const int8_t* qs = reinterpret_cast<const int8_t*>(qrow + (size_t)j * a.hq8);
                const float fj = fb[j];
                for (int e = 0; e < per; ++e) acc[e] += (float)qs[e] * fj;
            }
        }
    }
    float* dst = a.n_chunks == 1 ? a.out + (size_t)h * a.hs + i0
                                 : a.part_acc + ((size_t)h * a.n_chunks + c) * a.hs + i0;
    if (act)
        for (int e = 0; e < per; ++e) dst[e] = acc[e];
}

// Sum of the chunk partials of every head in chunk order.  A kernel of its
// own: a cross-workgroup handoff inside the values kernel would need
// device-scope fences, which write back L2 on this GPU.
__global__ void __launch_bounds__(256) attn_combine_kernel(const float* __restrict__ part, int n_chunks, int hs,
                                                           float* __restrict__ out) {
    const int h = blockIdx.x;
    for (int i = threadIdx.x; i < hs; i += blockDim.x) {
        const float* p = part + (size_t)h * n_chunks * hs + i;
        float tot = 0.0f;
#pragma unroll 8
        for (int cc = 0; cc < n_chunks; ++cc) tot += p[(size_t)cc * hs];
        out[(size_t)h * hs + i] = tot;
    }
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

// Top-k selection exactly as generate_token performs it (c:4818-4848): the
// k slots start as logits[0..k); scanning i = k..n-1, logits[i] replaces the
// slot holding the current minimum (the lowest slot among equal minima) when
// it is strictly greater.  The final slot order matters to the reference's
// later arithmetic (its pre-sort sum and, with top_p >= 1, its CDF walk), so
// it is reproduced, not just the top-k set.  Kernel 1 computes the maximum of
// every group of 64 logits (indices >= k); kernel 2, one wave, walks the
// groups in order and only visits groups whose maximum beats the current
// minimum.
constexpr int kSlotsPerLane = 16;            // k <= 1024

__global__ void __launch_bounds__(1024) topk_groupmax_kernel(const float* __restrict__ l, int n, int k, int ng,
                                                             float* gmax) {
    const int g = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int i = 64 * g + lane;
    float v = (i >= k && i < n) ? l[i] : -INFINITY;
    v = wave_max(v);
    if (lane == 0 && g < ng) gmax[g] = v;
}

__device__ __forceinline__ bool slot_less(float v, int s, float bv, int bs) {
    return v < bv || (v == bv && s < bs);
}

__global__ void __launch_bounds__(64) topk_scan_kernel(const float* __restrict__ l, int n, int k,
                                                       const float* __restrict__ gmax, int ng, float* out_v,
                                                       int* out_i) {
    const int lane = threadIdx.x;
    float sv[kSlotsPerLane];
    int si[kSlotsPerLane];
#pragma unroll
    for (int j = 0; j < kSlotsPerLane; ++j) {
        const int s = lane + 64 * j;
        sv[j] = s < k ? l[s] : INFINITY;
        si[j] = s < k ? s : -1;
    }
    // current minimum over slots: (value, slot) with the lowest slot on ties
    auto find_min = [&](float& mv, int& ms) {
        float bv = INFINITY;
        int bs = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < kSlotsPerLane; ++j) {
            const int s = lane + 64 * j;
            if (s < k && slot_less(sv[j], s, bv, bs)) { bv = sv[j]; bs = s; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int os = __shfl_xor(bs, o, 64);
            if (slot_less(ov, os, bv, bs)) { bv = ov; bs = os; }
        }
        mv = bv;
        ms = bs;
    };
    float cur;
    int cur_slot;
    find_min(cur, cur_slot);
    for (int g0 = 0; g0 < ng; g0 += 64) {
        const float gm = (g0 + lane < ng) ? gmax[g0 + lane] : -INFINITY;
        uint64_t flagged = __ballot(gm > cur);
        while (flagged) {
            const int j = __ffsll((unsigned long long)flagged) - 1;
            flagged &= flagged - 1;
            if (!(__shfl(gm, j, 64) > cur)) continue;
            const int base = 64 * (g0 + j);
            const int i = base + lane;
            const float v = (i >= k && i < n) ? l[i] : -INFINITY;
            uint64_t cand = __ballot(v > cur);
            while (cand) {
                const int c = __ffsll((unsigned long long)cand) - 1;
                cand &= cand - 1;
                const float bv = __shfl(v, c, 64);
                if (bv > cur) {
                    if (lane == (cur_slot & 63)) {
#pragma unroll
                        for (int jj = 0; jj < kSlotsPerLane; ++jj)
                            if (jj == (cur_slot >> 6)) { sv[jj] = bv; si[jj] = base + c; }
                    }
                    find_min(cur, cur_slot);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kSlotsPerLane; ++j) {
        const int s = lane + 64 * j;
        if (s < k) { out_v[s] = sv[j]; out_i[s] = si[j]; }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
void launch_embed(const Mat& emb, int token, float* x, hipStream_t s) {
    launch_dequant(emb.type, emb.w + (size_t)token * emb.rb, emb.cols, x, s);
}

void launch_rmsnorm(const float* xin, float* xscale, float scale, const float* w, int n, float inv_n, float eps,
                    float* out, const XPrep* xp, int form, hipStream_t s) {
    const XQ8 q = xp ? xp->q8 : XQ8{};
    const XDig d = xp ? xp->dig : XDig{};
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, xin, xscale, scale, w, n, inv_n, eps, out, q, d,
                       xp ? form : 0);
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
    a.layer_off = x.layer_off;
    a.att = x.att;
    a.part_acc = x.part_acc;
    a.part_ms = x.part_ms;
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
    // LDS: per-head block factors [kv_mul][8][kTC], then the chunk's V rows
    // (+8 bytes of alignment slack)
    const size_t lds = (size_t)x.kv_mul * 8 * kTC * 4 + (size_t)kTC * x.hq8 + 8;
    hipLaunchKernelGGL(attn_values_kernel, grid, block, lds, s, a);
    L3P_HIP(hipGetLastError());
    if (a.n_chunks > 1) {
        hipLaunchKernelGGL(attn_combine_kernel, dim3(x.n_heads), dim3(std::min(256, (x.hs + 63) / 64 * 64)), 0, s,
                           (const float*)a.part_acc, a.n_chunks, a.hs, a.out);
        L3P_HIP(hipGetLastError());
    }
}

void launch_softcap(float* l, int n, float cap, hipStream_t s) {
    hipLaunchKernelGGL(softcap_kernel, dim3((n + 255) / 256), dim3(256), 0, s, l, n, cap);
    L3P_HIP(hipGetLastError());
}

int sample_groups(int n) { return (n + 63) / 64; }
int sample_max_k() { return 64 * kSlotsPerLane; }

void launch_argmax(const float* l, int n, int* out, hipStream_t s, float* cv, int* ci) {
    const int nb = 256;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(nb), dim3(1024), 0, s, l, n, cv, ci);
    L3P_HIP(hipGetLastError());
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, s, cv, ci, nb, out);
    L3P_HIP(hipGetLastError());
}

void launch_topk_slots(const float* l, int n, int k, float* gmax, float* out_v, int* out_i, hipStream_t s) {
    L3P_REQUIRE(k >= 1 && k <= 64 * kSlotsPerLane && k <= n, L3P_E_UNSUPPORTED, "sampler: top_k=%d outside [1, %d]",
                k, 64 * kSlotsPerLane);
    const int ng = sample_groups(n);
    hipLaunchKernelGGL(topk_groupmax_kernel, dim3((ng + 15) / 16), dim3(1024), 0, s, l, n, k, ng, gmax);
    L3P_HIP(hipGetLastError());
    hipLaunchKernelGGL(topk_scan_kernel, dim3(1), dim3(64), 0, s, l, n, k, gmax, ng, out_v, out_i);
    L3P_HIP(hipGetLastError());
}
