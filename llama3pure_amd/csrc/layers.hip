// layers.hip — the per-layer kernels around the GEMVs and GEMMs (gfx950):
// QK-norm + RoPE + Q8_0 KV write fused into split-position GQA attention over
// the Q8_0 KV cache, the Gemma post-norm residuals, the row kernels of a
// prompt batch (embedding, RMSNorm, activation), logit soft-cap and the
// sampler.  Arithmetic follows llama3pure-c-engine.c (cited per kernel); the
// library is built with -ffp-contract=off so elementwise expressions round
// exactly as the reference's scalar C does.
#include "dequant.h"
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

// Q8_0 quantization with one value per lane, 32 lanes per block: the
// reference's quantize_row_q8_0 (c:1508-1528) per element.  Returns the
// quant; dh is the block's truncated fp16 scale (the same in its 32 lanes).
__device__ __forceinline__ int8_t quant_lane(float v, uint32_t& dh) {
    float amax = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;
    dh = f2h_trunc(d);
    int qi = (int)roundf(v * id);
    qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
    return (int8_t)qi;
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


// x += rmsnorm(y) (Gemma post-attention / post-FFN norm then residual,
// c:3364-3371, c:3411-3417), one row per workgroup (row strides ldy, ldx).
__global__ void __launch_bounds__(1024) rmsnorm_add_kernel(const float* __restrict__ y, int ldy,
                                                           const float* __restrict__ w, int n, float inv_n, float eps,
                                                           float* x, int ldx) {
    __shared__ float sh[16];
    const int t = threadIdx.x, nt = blockDim.x;
    y += (size_t)blockIdx.x * ldy;
    x += (size_t)blockIdx.x * ldx;
    float ss = 0.0f;
    for (int j = t; j < n; j += nt) ss += y[j] * y[j];
    ss = block_sum(ss, sh);
    const float r = 1.0f / sqrtf(ss * inv_n + eps);
    for (int j = t; j < n; j += nt) x[j] += w[j] * (r * y[j]);
}

// ---------------------------------------------------------------------------
// Rows of a prompt batch (transformer_prefill, c:3439-3680).
// ---------------------------------------------------------------------------
// x[b] = embedding row of tokens[b] (dequantize_row, c:3447-3452), times
// scale when non-zero (Gemma, c:3132-3148), and the step record
// {token, start + b} that token b's attention reads.
__global__ void embed_rows_kernel(int type, const uint8_t* __restrict__ emb, size_t rb, int n, float scale,
                                  const int* __restrict__ tokens, int start, float* __restrict__ x, int ldx,
                                  int* __restrict__ steps) {
    const int b = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    const int tok = tokens[b];
    if (i < n) {
        const float v = deq_elem(type, emb + (size_t)tok * rb, i);
        x[(size_t)b * ldx + i] = scale != 0.0f ? v * scale : v;
    }
    if (i == 0) {
        steps[2 * b] = tok;
        steps[2 * b + 1] = start + b;
    }
}

// o[b] = w * (r * x[b]) with r = 1/sqrt(sum(x[b]^2)/n + eps) (rmsnorm,
// c:3117-3129), one row per workgroup.
__global__ void __launch_bounds__(1024) rmsnorm_rows_kernel(const float* __restrict__ x, int ldx,
                                                            const float* __restrict__ w, int n, float inv_n,
                                                            float eps, float* __restrict__ o, int ldo) {
    __shared__ float sh[16];
    const int t = threadIdx.x, nt = blockDim.x;
    x += (size_t)blockIdx.x * ldx;
    o += (size_t)blockIdx.x * ldo;
    float ss = 0.0f;
    for (int j = t; j < n; j += nt) ss += x[j] * x[j];
    ss = block_sum(ss, sh);
    const float r = 1.0f / sqrtf(ss * inv_n + eps);
    for (int j = t; j < n; j += nt) o[j] = w[j] * (r * x[j]);
}

// h = act(h) * h2 elementwise over the batch's FFN rows: SwiGLU
// (c:3400-3406) or tanh-GeLU (c:3391-3398).
__global__ void act_rows_kernel(float* __restrict__ h, const float* __restrict__ h2, int64_t n, int gelu) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = gelu ? ref_geglu(h[i], h2[i]) : ref_swiglu(h[i], h2[i]);
}

// ---------------------------------------------------------------------------
// Attention of one decode step over the Q8_0 KV cache (c:3232-3359), as
// flash-decoding over chunks of kTC positions.  attn_chunk_kernel: workgroup
// = one KV group (kv_mul waves, one per query head) x one chunk:
//   * Gemma QK-norm (c:3151-3165), RoPE with attn_scale fused into Q
//     (c:3240-3296) and Q8_0 quantization of Q (c:3311-3312) for the
//     group's query heads; the chunk holding the step's position also
//     quantizes K and V into the cache there (c:3301-3308);
//   * the chunk's K and V rows are copied HBM -> LDS;
//   * scores are the reference's dot_q8_0_q8_0_cache (c:1574-1597): exact
//     integer block dots summed in fp32 in block order (bit-exact);
//   * the chunk's softmax max m and sum l of e = expf(s - m), and the
//     unnormalized V accumulation sum_t q_t * (d_t * e_t) (accum_q8_0_cache,
//     c:1600-1622).  A position is skipped when e < 1e-8: its normalized
//     weight expf(s - M) / S is then below 1e-8 too, the reference's skip
//     threshold (c:1602).
// attn_merge_kernel then forms the reference's softmax max M and sum S from
// the chunk statistics (softmax, c:3167-3186) and the output
// sum_c acc_c * expf(m_c - M) / S.
// ---------------------------------------------------------------------------
struct AttnCArgs {
    const float *q, *k, *v;          // this step's projections [heads][hs]
    const float *q_norm, *k_norm;    // Gemma QK-norm weights (null otherwise)
    const float *cos, *sin;          // RoPE tables [seq][hs/2]; the step's row is used
    uint8_t *kc, *vc;                // this layer's caches [n_kv][seq][hq8]
    const int* step;                 // device {token, pos}
    float* part;                     // [n_heads][n_chunks][hs + 2]: chunk output, max, sum
    float* out;                      // [n_heads][hs]
    size_t head_seq;
    int n_heads, kv_mul, hs, hq8, window, neox;
    float attn_scale, eps, inv_hs;
    // Prompt batches: token z (the last grid dimension) uses q + z*q_stride,
    // k, v + z*kv_stride, step + 2z, part + z*part_stride, out + z*out_stride,
    // and its K/V rows are already in the cache (kv_ready, kv_rows_kernel).
    int q_stride, kv_stride, out_stride, kv_ready;
    size_t part_stride;
};

// The arguments of token z of a prompt batch (z = 0: a decode step).
__device__ __forceinline__ AttnCArgs token_args(const AttnCArgs& a0, int z) {
    AttnCArgs a = a0;
    a.q += (size_t)z * a.q_stride;
    a.k += (size_t)z * a.kv_stride;
    a.v += (size_t)z * a.kv_stride;
    a.step += 2 * z;
    a.part += (size_t)z * a.part_stride;
    a.out += (size_t)z * a.out_stride;
    return a;
}

// Positions this step attends to: [t0, pos], in chunks of kTC (c:3316-3322).
struct Span {
    int pos, t0, na, n_chunks;
};
__device__ __forceinline__ Span span_of(const int* step, int window) {
    Span s;
    s.pos = step[1];
    s.t0 = window > 0 ? max(0, s.pos - window + 1) : 0;
    s.na = s.pos - s.t0 + 1;
    s.n_chunks = (s.na + kTC - 1) / kTC;
    return s;
}

// Q8_0 block `b` of a cache row starting at byte offset `off` of a dword
// array (LDS here): fp16 scale and the 32 quants as eight dwords.
__device__ __forceinline__ float row_block(const uint32_t* base, uint32_t off, uint32_t (&q)[8]) {
    const uint32_t E = off >> 2;
    const bool odd = (off & 2u) != 0;   // block starts 2 bytes into a dword
    uint32_t dw[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) dw[k] = base[E + k];
    // quants: dwords E+1.. when odd, two bytes into dword E otherwise
#pragma unroll
    for (int k = 0; k < 8; ++k) q[k] = odd ? dw[k + 1] : __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2);
    return h2f(odd ? (dw[0] >> 16) : dw[0]);
}

__global__ void __launch_bounds__(1024) attn_chunk_kernel(AttnCArgs a0) {
    extern __shared__ __align__(16) float smem[];
    const AttnCArgs a = token_args(a0, blockIdx.z);
    const int g = blockIdx.x, c = blockIdx.y;
    const Span sp = span_of(a.step, a.window);
    if (c >= sp.n_chunks) return;   // the grid covers the longest context
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nt = blockDim.x;
    const int hs = a.hs, nb = hs / 32, half = hs / 2, km = a.kv_mul;
    const int h = g * km + w;
    const int jbeg = c * kTC, jend = min(sp.na, jbeg + kTC), cnt = jend - jbeg;
    // the chunk holding the step's position forms and writes its K/V row,
    // unless a prompt batch's kv_rows_kernel already wrote it
    const bool has_pos = c == sp.n_chunks - 1 && !a.kv_ready;

    // LDS: [kv_mul][hs] q rows, [2][hs] k and v rows, [kv_mul][8][kTC] V
    // factors, [kv_mul][hs] int8 q, [kv_mul][8] q scales, then the chunk's K
    // rows and V rows (kTC * hq8 bytes + 8 each, dword aligned)
    float* qh = smem;
    float* kvh = qh + km * hs;
    float* f = kvh + 2 * hs;
    int8_t* qq = reinterpret_cast<int8_t*>(f + km * 8 * kTC);
    float* qd = reinterpret_cast<float*>(qq + km * hs);
    const int rowdw = (kTC * a.hq8 + 8 + 3) / 4;
    uint32_t* krows = reinterpret_cast<uint32_t*>(qd + km * 8);
    uint32_t* vrows = krows + rowdw;

    // this step's q (and k, v) rows, RoPE factors and norm weights go to
    // registers first: everything is issued before the row copies below, so
    // waiting for these loads never waits for the copies (hs <= 256)
    const float* cosr = a.cos + (size_t)sp.pos * half;
    const float* sinr = a.sin + (size_t)sp.pos * half;
    float qv[4], kv2[8], cs[2], sn[2], qn[4], kn[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = lane + 64 * k;
        qv[k] = j < hs ? a.q[(size_t)h * hs + j] : 0.0f;
        qn[k] = (a.q_norm && j < hs) ? a.q_norm[j] : 0.0f;
        kn[k] = (a.k_norm && j < hs) ? a.k_norm[j] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int p = lane + 64 * k;
        cs[k] = p < half ? cosr[p] : 0.0f;
        sn[k] = p < half ? sinr[p] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {   // k then v over the workgroup (2*hs <= 8*64)
        const int j = threadIdx.x + nt * k;
        kv2[k] = (has_pos && j < 2 * hs) ? (j < hs ? a.k[(size_t)g * hs + j] : a.v[(size_t)g * hs + j - hs]) : 0.0f;
    }

    // the chunk's K and V rows, HBM -> LDS (dword copies from the 4-byte
    // aligned start; the row at the step's position is replaced below)
    const size_t start = (size_t)g * a.head_seq + (size_t)(sp.t0 + jbeg) * a.hq8;
    const size_t s4 = start & ~(size_t)3;
    const int nd = (int)((start + (size_t)cnt * a.hq8 - s4 + 3) >> 2);
    {
        const uint32_t* ks = reinterpret_cast<const uint32_t*>(a.kc) + (s4 >> 2);
        const uint32_t* vs = reinterpret_cast<const uint32_t*>(a.vc) + (s4 >> 2);
        const int nw = nt >> 6;
        for (int i = w; i * 64 < nd; i += nw) {
            if (i * 64 + lane < nd) {
                __builtin_amdgcn_global_load_lds(ks + i * 64 + lane, (lds_void*)(krows + i * 64), 4, 0, 0);
                __builtin_amdgcn_global_load_lds(vs + i * 64 + lane, (lds_void*)(vrows + i * 64), 4, 0, 0);
            }
        }
    }
    const uint32_t roff = (uint32_t)(start - s4);   // byte offset of row 0 in krows / vrows

    // QK-norm + RoPE + Q8_0 of the group's query heads (and of K, V at pos)
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (lane + 64 * k < hs) qh[w * hs + lane + 64 * k] = qv[k];
    if (has_pos)
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (threadIdx.x + nt * k < 2 * hs) kvh[threadIdx.x + nt * k] = kv2[k];
    __syncthreads();
    if (a.q_norm) {   // per-head rmsnorm (c:3151-3165); every wave also forms K's factor
        float ssq = 0.0f, ssk = 0.0f;
        for (int j = lane; j < hs; j += 64) {
            ssq += qh[w * hs + j] * qh[w * hs + j];
            ssk += kvh[j] * kvh[j];
        }
        ssq = wave_sum(ssq);
        ssk = wave_sum(ssk);
        const float rq = 1.0f / sqrtf(ssq * a.inv_hs + a.eps);
        const float rk = 1.0f / sqrtf(ssk * a.inv_hs + a.eps);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = lane + 64 * k;
            if (j < hs) {
                qh[w * hs + j] = qn[k] * (rq * qh[w * hs + j]);
                if (has_pos && w == 0) kvh[j] = kn[k] * (rk * kvh[j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {   // RoPE: NEOX (Gemma) or interleaved pairs
        const int p = lane + 64 * k;
        if (p < half) {
            const int i0 = a.neox ? p : 2 * p;
            const int i1 = a.neox ? p + half : 2 * p + 1;
            const float v0 = qh[w * hs + i0], v1 = qh[w * hs + i1];
            qh[w * hs + i0] = (v0 * cs[k] - v1 * sn[k]) * a.attn_scale;
            qh[w * hs + i1] = (v0 * sn[k] + v1 * cs[k]) * a.attn_scale;
            if (has_pos && w == 0) {
                const float k0 = kvh[i0], k1 = kvh[i1];
                kvh[i0] = k0 * cs[k] - k1 * sn[k];
                kvh[i1] = k0 * sn[k] + k1 * cs[k];
            }
        }
    }
    __syncthreads();
    // Q8_0 of the head's q, one value per lane (c:3311-3312)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = lane + 64 * k;
        if (k * 64 < hs) {
            uint32_t dh;
            const int8_t qv8 = quant_lane(j < hs ? qh[w * hs + j] : 0.0f, dh);   // all lanes take part
            if (j < hs) {
                qq[w * hs + j] = qv8;
                if ((lane & 31) == 0) qd[w * 8 + (j >> 5)] = h2f_exact(dh);
            }
        }
    }
    // K (wave 0) and V (wave 1, or 0 for one-wave groups) of the step, quantized
    // here one value per lane; the copy replaces the copied row in LDS and goes
    // to the cache at the end of the kernel (c:3301-3308)
    const int kvsel = w == 0 ? 0 : (w == 1 ? 1 : -1);
    const bool kv_wave = has_pos && (kvsel >= 0 || km == 1);
    uint32_t kvq[2][4], kvdh[2][4];
    if (kv_wave) {
#pragma unroll
        for (int sel = 0; sel < 2; ++sel) {
            if (km > 1 && sel != kvsel) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (k * 64 < hs)
                    kvq[sel][k] = (uint8_t)quant_lane(lane + 64 * k < hs ? kvh[sel * hs + lane + 64 * k] : 0.0f,
                                                      kvdh[sel][k]);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0): this wave's row copies have landed
    __syncthreads();
    if (kv_wave) {   // the step's own K/V row replaces the copied one
#pragma unroll
        for (int sel = 0; sel < 2; ++sel) {
            if (km > 1 && sel != kvsel) continue;
            uint8_t* rb = reinterpret_cast<uint8_t*>(sel ? vrows : krows) + roff + (size_t)(cnt - 1) * a.hq8;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int j = lane + 64 * k;
                if (j < hs) {
                    const int b = j >> 5;
                    rb[34 * b + 2 + (j & 31)] = (uint8_t)kvq[sel][k];
                    if ((lane & 31) == 0) {
                        rb[34 * b] = (uint8_t)(kvdh[sel][k] & 0xff);
                        rb[34 * b + 1] = (uint8_t)(kvdh[sel][k] >> 8);
                    }
                }
            }
        }
    }
    __syncthreads();

    // scores of head h: lane = position
    float sc = -INFINITY;
    if (lane < cnt) {
        float sum = 0.0f;
        const int8_t* qw = qq + w * hs;
        for (int b = 0; b < nb; ++b) {
            uint32_t kq[8];
            const float db = row_block(krows, roff + (uint32_t)lane * a.hq8 + 34u * b, kq);
            int isum = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                isum = __builtin_amdgcn_sdot4(*reinterpret_cast<const int*>(qw + 32 * b + 4 * k), (int)kq[k], isum, false);
            sum += qd[w * 8 + b] * db * (float)isum;
        }
        sc = sum;
    }
    const float m = wave_max(sc);
    const float e = lane < cnt ? expf(sc - m) : 0.0f;
    const float l = wave_sum(e);

    // f[b][j] = d(V row j, block b) * e_j, 0 for skipped positions
    const uint8_t* vbytes = reinterpret_cast<const uint8_t*>(vrows) + roff;
    float* fw = f + (size_t)w * 8 * kTC;
    if (lane < cnt) {
        const bool skip = e < 1e-8f;
        for (int bb = 0; bb < nb; ++bb) {
            const uint8_t* s2 = vbytes + (size_t)lane * a.hq8 + 34 * bb;
            const float d = h2f((uint32_t)s2[0] | ((uint32_t)s2[1] << 8));
            fw[bb * kTC + lane] = skip ? 0.0f : d * e;
        }
    }
    __syncthreads();
    const int per = (hs + 63) / 64;            // outputs per lane (1, 2 or 4)
    const int i0 = lane * per;
    const bool act = i0 < hs;
    const int b = act ? i0 >> 5 : 0;
    const uint8_t* qrow = vbytes + 34 * b + 2 + (i0 & 31);
    const float* fb = fw + b * kTC;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
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
                for (int e2 = 0; e2 < per; ++e2) acc[e2] += (float)qs[e2] * fj;
            }
        }
    }
    float* dst = a.part + ((size_t)h * sp.n_chunks + c) * (hs + 2);
    if (act)
        for (int e2 = 0; e2 < per; ++e2) dst[i0 + e2] = acc[e2];
    if (lane == 0) {
        dst[hs] = m;
        dst[hs + 1] = l;
    }
    if (kv_wave) {   // K and V of the step into the cache (c:3301-3308)
#pragma unroll
        for (int sel = 0; sel < 2; ++sel) {
            if (km > 1 && sel != kvsel) continue;
            uint8_t* cd = (sel ? a.vc : a.kc) + (size_t)g * a.head_seq + (size_t)sp.pos * a.hq8;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int j = lane + 64 * k;
                if (j < hs) {
                    const int b = j >> 5;
                    cd[34 * b + 2 + (j & 31)] = (uint8_t)kvq[sel][k];
                    if ((lane & 31) == 0) {
                        cd[34 * b] = (uint8_t)(kvdh[sel][k] & 0xff);
                        cd[34 * b + 1] = (uint8_t)(kvdh[sel][k] >> 8);
                    }
                }
            }
        }
    }
}

// K and V rows of every token of a prompt batch into the cache, before the
// batch's attention reads them (c:3301-3308): for KV head g = blockIdx.x of
// token z = blockIdx.y, Gemma's QK-norm of k (c:3232-3236), RoPE of k
// (c:3254-3296) and the Q8_0 rows of k and v (quantize_to_q8_0_cache,
// c:1535-1570), with the arithmetic and order of attn_chunk_kernel's own
// K/V path.  One wave.
__global__ void __launch_bounds__(64) kv_rows_kernel(AttnCArgs a0) {
    __shared__ float kvh[2 * 256];
    const AttnCArgs a = token_args(a0, blockIdx.y);
    const int g = blockIdx.x, lane = threadIdx.x;
    const int hs = a.hs, half = hs / 2;
    const int pos = a.step[1];
    for (int j = lane; j < 2 * hs; j += 64)
        kvh[j] = j < hs ? a.k[(size_t)g * hs + j] : a.v[(size_t)g * hs + j - hs];
    __syncthreads();
    if (a.k_norm) {
        float ssk = 0.0f;
        for (int j = lane; j < hs; j += 64) ssk += kvh[j] * kvh[j];
        ssk = wave_sum(ssk);
        const float rk = 1.0f / sqrtf(ssk * a.inv_hs + a.eps);
        __syncthreads();
        for (int j = lane; j < hs; j += 64) kvh[j] = a.k_norm[j] * (rk * kvh[j]);
        __syncthreads();
    }
    const float* cosr = a.cos + (size_t)pos * half;
    const float* sinr = a.sin + (size_t)pos * half;
    for (int p = lane; p < half; p += 64) {
        const int i0 = a.neox ? p : 2 * p;
        const int i1 = a.neox ? p + half : 2 * p + 1;
        const float k0 = kvh[i0], k1 = kvh[i1], cs = cosr[p], sn = sinr[p];
        kvh[i0] = k0 * cs - k1 * sn;
        kvh[i1] = k0 * sn + k1 * cs;
    }
    __syncthreads();
#pragma unroll
    for (int sel = 0; sel < 2; ++sel) {
        uint8_t* cd = (sel ? a.vc : a.kc) + (size_t)g * a.head_seq + (size_t)pos * a.hq8;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = lane + 64 * k;
            if (k * 64 < hs) {
                uint32_t dh;
                const int8_t q = quant_lane(j < hs ? kvh[sel * hs + j] : 0.0f, dh);   // all lanes take part
                if (j < hs) {
                    const int b = j >> 5;
                    cd[34 * b + 2 + (j & 31)] = (uint8_t)q;
                    if ((lane & 31) == 0) {
                        cd[34 * b] = (uint8_t)(dh & 0xff);
                        cd[34 * b + 1] = (uint8_t)(dh >> 8);
                    }
                }
            }
        }
    }
}

// out = sum_c acc_c * expf(m_c - M) / S with M = max m_c, S = sum l_c expf(m_c - M).
// Every load is issued before anything waits: the first wave reads the
// chunk maxima and sums (lane = chunk) while each thread reads its output's
// chunk partials; the weights expf(m_c - M) / S go through LDS.
__global__ void __launch_bounds__(256) attn_merge_kernel(AttnCArgs a0) {
    __shared__ float wc[256];
    const AttnCArgs a = token_args(a0, blockIdx.y);
    const Span sp = span_of(a.step, a.window);
    const int h = blockIdx.x, hs = a.hs, nch = sp.n_chunks, t = threadIdx.x;
    const float* part = a.part + (size_t)h * nch * (hs + 2);
    for (int c0 = 0; c0 < nch; c0 += 64) {   // 64 chunks (4096 positions) per round
        const int nc = min(64, nch - c0);
        float pv[64];
        const int i = t;   // this thread's output element (hs <= 256 = blockDim)
#pragma unroll
        for (int k = 0; k < 64; ++k) pv[k] = (k < nc && i < hs) ? part[(size_t)(c0 + k) * (hs + 2) + i] : 0.0f;
        if (t < 64) {
            const bool ok = t < nch;
            // the statistics of every chunk (not only this round's), for M and S
            float mx = -INFINITY;
            for (int c = t; c < nch; c += 64) mx = fmaxf(mx, part[(size_t)c * (hs + 2) + hs]);
            mx = wave_max(mx);
            float ssum = 0.0f;
            for (int c = t; c < nch; c += 64) {
                const float* pc = part + (size_t)c * (hs + 2);
                ssum += pc[hs + 1] * expf(pc[hs] - mx);
            }
            ssum = wave_sum(ssum);
            const float inv = 1.0f / ssum;
            if (t < nc) wc[t] = expf(part[(size_t)(c0 + t) * (hs + 2) + hs] - mx) * inv;
            (void)ok;
        }
        __syncthreads();
        if (i < hs) {
            float tot = c0 == 0 ? 0.0f : a.out[(size_t)h * hs + i];
#pragma unroll
            for (int k = 0; k < 64; ++k)
                if (k < nc) tot += pv[k] * wc[k];
            a.out[(size_t)h * hs + i] = tot;
        }
        __syncthreads();
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
void launch_embed_step(const Mat& emb, int token, int pos, float scale, float* x, int* step, hipStream_t s) {
    launch_embed_row(emb.type, emb.w + (size_t)token * emb.rb, emb.cols, scale, x, token, pos, step, s);
}

void launch_rmsnorm_add(const float* y, const float* w, int n, float inv_n, float eps, float* x, hipStream_t s) {
    launch_rmsnorm_add_rows(y, 0, w, n, inv_n, eps, x, 0, 1, s);
}

void launch_rmsnorm_add_rows(const float* y, int ldy, const float* w, int n, float inv_n, float eps, float* x,
                             int ldx, int rows, hipStream_t s) {
    if (rows == 0) return;
    hipLaunchKernelGGL(rmsnorm_add_kernel, dim3(rows), dim3(1024), 0, s, y, ldy, w, n, inv_n, eps, x, ldx);
    L3P_HIP(hipGetLastError());
}

void launch_embed_rows(const Mat& emb, const int* tokens, int rows, int start, float scale, float* x, int ldx,
                       int* steps, hipStream_t s) {
    if (rows == 0) return;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((emb.cols + 255) / 256, rows), dim3(256), 0, s, emb.type, emb.w,
                       emb.rb, emb.cols, scale, tokens, start, x, ldx, steps);
    L3P_HIP(hipGetLastError());
}

void launch_rmsnorm_rows(const float* x, int ldx, const float* w, int n, float inv_n, float eps, float* o, int ldo,
                         int rows, hipStream_t s) {
    if (rows == 0) return;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(1024), 0, s, x, ldx, w, n, inv_n, eps, o, ldo);
    L3P_HIP(hipGetLastError());
}

void launch_act_rows(float* h, const float* h2, int64_t n, bool gelu, hipStream_t s) {
    if (n == 0) return;
    hipLaunchKernelGGL(act_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, h, h2, n, gelu ? 1 : 0);
    L3P_HIP(hipGetLastError());
}

void launch_attention(const Model& m, int l, float* out, hipStream_t s) {
    launch_attention(m, l, AttnIO{m.q, m.k, m.v, m.step, out}, s);
}

// The attention arguments of layer l for the token whose rows io holds.
static AttnCArgs attn_args(const Model& m, int l, const AttnIO& io) {
    const Layer& L = m.layers[l];
    const bool swa = m.swa_pattern > 0 && (l % m.swa_pattern < m.swa_pattern - 1);   // c:3247
    const bool use_swa = m.is_gemma && swa;
    AttnCArgs a{};
    a.q = io.q;
    a.k = io.k;
    a.v = io.v;
    a.q_norm = m.is_gemma ? L.q_norm : nullptr;
    a.k_norm = m.is_gemma ? L.k_norm : nullptr;
    a.cos = use_swa ? m.cos_s : m.cos_d;
    a.sin = use_swa ? m.sin_s : m.sin_d;
    a.kc = m.kc + (size_t)l * m.layer_kv;
    a.vc = m.vc + (size_t)l * m.layer_kv;
    a.step = io.step;
    a.part = m.part_acc;
    a.out = io.out;
    a.head_seq = m.head_seq;
    a.n_heads = m.n_heads;
    a.kv_mul = m.kv_mul;
    a.hs = m.hs;
    a.hq8 = m.hq8;
    a.window = (use_swa && m.swa_window > 0) ? m.swa_window : 0;   // c:3316-3321
    a.neox = m.is_gemma;
    a.attn_scale = m.attn_scale;
    a.eps = m.eps > 0 ? m.eps : 1e-5f;
    a.inv_hs = m.inv_hs;
    return a;
}

// Chunk and merge launches for `tokens` tokens of up to `chunks` chunks each.
static void launch_chunks(const Model& m, const AttnCArgs& a, int chunks, int tokens, hipStream_t s) {
    const int rowdw = (kTC * m.hq8 + 8 + 3) / 4;
    const size_t lds = (size_t)m.kv_mul * m.hs * 4 + 2 * (size_t)m.hs * 4 + (size_t)m.kv_mul * 8 * kTC * 4 +
                       (size_t)m.kv_mul * m.hs + (size_t)m.kv_mul * 8 * 4 + 2 * (size_t)rowdw * 4 + 16;
    const dim3 grid(m.n_kv, chunks, tokens), block(64 * m.kv_mul);
    static size_t lds_set = 65536;   // dynamic LDS above 64 KB must be allowed first
    if (lds > lds_set) {
        L3P_HIP(hipFuncSetAttribute((const void*)attn_chunk_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        lds_set = lds;
    }
    hipLaunchKernelGGL(attn_chunk_kernel, grid, block, lds, s, a);
    L3P_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_merge_kernel, dim3(m.n_heads, tokens), dim3((m.hs + 63) / 64 * 64), 0, s, a);
    L3P_HIP(hipGetLastError());
}

void launch_attention(const Model& m, int l, const AttnIO& io, hipStream_t s) {
    launch_chunks(m, attn_args(m, l, io), m.max_chunks, 1, s);
}

int attention_chunks(const Model& m, int l, int last_pos) {
    const AttnCArgs a = attn_args(m, l, AttnIO{});
    const int t0 = a.window > 0 ? std::max(0, last_pos - a.window + 1) : 0;
    return (last_pos - t0 + 1 + kTC - 1) / kTC;
}

void launch_attention_rows(const Model& m, int l, const AttnIO& io, int q_stride, int kv_stride, int out_stride,
                           int tokens, int last_pos, float* part, size_t part_cap, hipStream_t s) {
    if (tokens == 0) return;
    AttnCArgs a = attn_args(m, l, io);
    const int chunks = attention_chunks(m, l, last_pos);   // the most any token of the batch has
    a.q_stride = q_stride;
    a.kv_stride = kv_stride;
    a.out_stride = out_stride;
    a.kv_ready = 1;
    a.part = part;
    a.part_stride = (size_t)m.n_heads * chunks * (m.hs + 2);
    L3P_REQUIRE(a.part_stride * tokens <= part_cap, L3P_E_INVALID, "attention: %d tokens exceed the partials buffer",
                tokens);
    hipLaunchKernelGGL(kv_rows_kernel, dim3(m.n_kv, tokens), dim3(64), 0, s, a);
    L3P_HIP(hipGetLastError());
    launch_chunks(m, a, chunks, tokens, s);
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
