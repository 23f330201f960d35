// layers.hip — the per-layer kernels around the GEMVs and GEMMs (gfx950):
// QK-norm + RoPE + Q8_0 KV write fused into split-position GQA attention over
// the Q8_0 KV cache, the Gemma post-norm residuals, the row kernels of a
// prompt batch (embedding, RMSNorm, activation), logit soft-cap and the
// sampler.  Arithmetic follows llama3pure-c-engine.c (cited per kernel); the
// library is built with -ffp-contract=off so elementwise expressions round
// exactly as the reference's scalar C does.
#include <string.h>

#include "dequant.h"
#include "device_common.h"
#include "model.h"

namespace {

constexpr int kTC = 64;   // positions per attention chunk (one per lane); decode steps of
                          // models with head_dim >= 192 use 32 (Model::dec_tc)
typedef __attribute__((address_space(3))) void lds_void;

using namespace l3pd;

// Q8_0 quantization with one value per lane, 32 lanes per block: the
// reference's quantize_row_q8_0 (c:1508-1528) per element.  Returns the
// quant; dh is the block's truncated fp16 scale (the same in its 32 lanes).
__device__ __forceinline__ int8_t quant_lane(float v, uint32_t& dh) {
    const float amax = half_max(fabsf(v));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;
    dh = f2h_trunc(d);
    int qi = (int)roundf(v * id);
    qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
    return (int8_t)qi;
}

// quant_lane on N values per lane at once (value k of lane l is element
// l + 64 k of a row): the same arithmetic, with the N reductions and
// divisions interleaved instead of run one after another.
template <int N>
__device__ __forceinline__ void quant_lanes(const float (&v)[N], int8_t (&q)[N], uint32_t (&dh)[N]) {
    float a[N];
#pragma unroll
    for (int k = 0; k < N; ++k) a[k] = fabsf(v[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) a[k] = fmaxf(a[k], lane_partner<16>(a[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) a[k] = fmaxf(a[k], lane_partner<8>(a[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) a[k] = fmaxf(a[k], lane_partner<4>(a[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) a[k] = fmaxf(a[k], lane_partner<2>(a[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) a[k] = fmaxf(a[k], lane_partner<1>(a[k]));
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const float d = a[k] / 127.0f;
        const float id = d > 0.0f ? 127.0f / a[k] : 0.0f;
        dh[k] = f2h_trunc(d);
        int qi = (int)roundf(v[k] * id);
        qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
        q[k] = (int8_t)qi;
    }
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [LO, HI], by binary search over
// the immediate forms
template <int LO, int HI>
__device__ __forceinline__ void wait_vm_dyn(int n) {
    if constexpr (LO == HI) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LO) : "memory");
    } else {
        constexpr int MID = (LO + HI) / 2;
        if (n <= MID) wait_vm_dyn<LO, MID>(n);
        else wait_vm_dyn<MID + 1, HI>(n);
    }
}
__device__ __forceinline__ void wait_vm_upto(int n) { wait_vm_dyn<0, 63>(n < 63 ? n : 63); }

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
    const float* rope;               // decode steps: the step's cos row then sin row (null: read the tables)
    uint8_t *kc, *vc;                // this layer's caches [n_kv][seq][hq8]
    const int* step;                 // device {token, pos}
    float* part;                     // [n_heads][part_chunks][attn_part_row(hs)]: chunk output, max, sum
    int part_chunks;                 // chunk slots per head in part
    int tc;                          // positions per chunk (kTC or 32)
    float* out;                      // [n_heads][hs]
    size_t head_seq;
    int n_heads, kv_mul, hs, hq8, window, neox;
    float attn_scale, eps, inv_hs;
    // Prompt batches: token z (the last grid dimension) uses q + z*q_stride,
    // k, v + z*kv_stride, step + 2z, part + z*part_stride, out + z*out_stride,
    // and its K/V rows are already in the cache (kv_ready, kv_rows_kernel).
    int q_stride, kv_stride, out_stride, kv_ready;
    size_t part_stride;
    float softcap;   // > 0: scores s -> softcap * tanhf(s / softcap) (a load option; 0: none)
};

// A score after the optional cap (attention logit soft-capping).
__device__ __forceinline__ float cap_score(float s, float cap) {
    return cap > 0.0f ? cap * tanhf(s / cap) : s;
}

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

// Positions this step attends to: [t0, pos], in chunks of tc (c:3316-3322).
struct Span {
    int pos, t0, na, n_chunks;
};
__device__ __forceinline__ Span span_at(int pos, int window, int tc) {
    Span s;
    s.pos = pos;
    s.t0 = window > 0 ? max(0, s.pos - window + 1) : 0;
    s.na = s.pos - s.t0 + 1;
    s.n_chunks = (s.na + tc - 1) / tc;
    return s;
}
__device__ __forceinline__ Span span_of(const int* step, int window, int tc) { return span_at(step[1], window, tc); }

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

// V values of one cache row for the lane's PER outputs (PER consecutive bytes
// inside one 32-block, 2-byte aligned for PER >= 2)
template <int PER>
__device__ __forceinline__ uint32_t v_quants(const uint8_t* p) {
    if (PER == 1) return *p;
    if (PER == 2) return *reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)reinterpret_cast<const uint16_t*>(p)[0] | ((uint32_t)reinterpret_cast<const uint16_t*>(p)[1] << 16);
}

// acc += q * (d * e) for the lane's PER outputs, the position skipped when
// e < 1e-8 (accum_q8_0_cache, c:1600-1622)
template <int PER>
__device__ __forceinline__ void v_accum(uint32_t dh, uint32_t q, float e, float (&acc)[4]) {
    const float f = e < 1e-8f ? 0.0f : h2f(dh) * e;
#pragma unroll
    for (int i = 0; i < PER; ++i) acc[i] = fmaf((float)(int8_t)((q >> (8 * i)) & 0xffu), f, acc[i]);
}

// One 16-byte piece per lane into LDS (lane i of the instruction writes dst + 16 i).
__device__ __forceinline__ void piece16(const uint8_t* src, uint32_t* dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 16, 0, 0);
}

// Dwords of LDS for one chunk's K (or V) rows: TC rows of hq8 bytes copied
// in 16-byte pieces from the 16-byte aligned address at or below the first
// row (up to 15 bytes before it and 15 after the last row).
__host__ __device__ constexpr int chunk_rows_dw(int tc, int hq8) { return 4 * ((tc * hq8 + 30) / 16 + 1); }

template <int NB, int TC>
__global__ void __launch_bounds__(1024) attn_chunk_kernel(AttnCArgs a0) {
    extern __shared__ __align__(16) float smem[];
    const AttnCArgs a = token_args(a0, blockIdx.z);
    const int g = blockIdx.x, c = blockIdx.y;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, nt = blockDim.x;
    constexpr int hs = 32 * NB, half = hs / 2, hq8 = 34 * NB;
    constexpr int NQ = (hs + 63) / 64;     // elements of a head row per lane
    constexpr int NR = (half + 63) / 64;   // RoPE factors per lane
    constexpr int PER = NB <= 2 ? 1 : (NB <= 4 ? 2 : 4);   // V outputs per lane, inside one 32-block
    const int km = a.kv_mul;
    const int h = g * km + w;

    // LDS: [kv_mul][hs] q rows, [2][hs] k and v rows, [kv_mul][8][TC] V
    // factors, [kv_mul][hs] int8 q, [kv_mul][8] q scales, [2][hs] q and k norm
    // weights, [2][hs/2] RoPE cos and sin, then the chunk's K rows and V rows
    // (chunk_rows_dw dwords each); every part starts 16-byte aligned
    float* qh = smem;
    float* kvh = qh + km * hs;
    float* f = kvh + 2 * hs;
    int8_t* qq = reinterpret_cast<int8_t*>(f + km * 8 * TC);
    float* qd = reinterpret_cast<float*>(qq + km * hs);
    float* nrm = qd + km * 8;
    float* rope = nrm + 2 * hs;
    const int rowdw = chunk_rows_dw(TC, hq8);
    uint32_t* krows = reinterpret_cast<uint32_t*>(rope + hs);
    uint32_t* vrows = krows + rowdw;

    // this step's q, k and v rows, the norm weights and, for a decode step,
    // the RoPE factors of its position, HBM -> LDS in 16-byte pieces, and the
    // step record: none depends on another, so one wait covers them all.
    // Wave w copies its query head's row, wave 0 the group's k and v rows,
    // the norm weights and the RoPE factors.
    const bool row_lane = lane < hs / 4;
    if (row_lane) {
        piece16(reinterpret_cast<const uint8_t*>(a.q + (size_t)h * hs) + 16 * lane, reinterpret_cast<uint32_t*>(qh + w * hs));
        if (w == 0) {
            piece16(reinterpret_cast<const uint8_t*>(a.k + (size_t)g * hs) + 16 * lane, reinterpret_cast<uint32_t*>(kvh));
            piece16(reinterpret_cast<const uint8_t*>(a.v + (size_t)g * hs) + 16 * lane,
                    reinterpret_cast<uint32_t*>(kvh + hs));
            if (a.q_norm) {
                piece16(reinterpret_cast<const uint8_t*>(a.q_norm) + 16 * lane, reinterpret_cast<uint32_t*>(nrm));
                piece16(reinterpret_cast<const uint8_t*>(a.k_norm) + 16 * lane, reinterpret_cast<uint32_t*>(nrm + hs));
            }
        }
    }
    const bool rope_lane = w == 0 && lane < half / 4;
    if (a.rope && rope_lane) {
        piece16(reinterpret_cast<const uint8_t*>(a.rope) + 16 * lane, reinterpret_cast<uint32_t*>(rope));
        piece16(reinterpret_cast<const uint8_t*>(a.rope + half) + 16 * lane, reinterpret_cast<uint32_t*>(rope + half));
    }
    const int pos = *reinterpret_cast<const volatile int*>(a.step + 1);   // issued here, before the wait
    wait_vm_dyn<0, 0>(0);
    lds_sync();
    const Span sp = span_at(pos, a.window, a.tc);
    if (c >= sp.n_chunks) return;   // the grid covers the longest context
    const int jbeg = c * TC, jend = min(sp.na, jbeg + TC), cnt = jend - jbeg;
    // the chunk holding the step's position forms and writes its K/V row,
    // unless a prompt batch's kv_rows_kernel already wrote it
    const bool has_pos = c == sp.n_chunks - 1 && !a.kv_ready;

    // prompt batches: the RoPE factors of the token's position
    if (!a.rope && rope_lane) {
        piece16(reinterpret_cast<const uint8_t*>(a.cos + (size_t)sp.pos * half) + 16 * lane,
                reinterpret_cast<uint32_t*>(rope));
        piece16(reinterpret_cast<const uint8_t*>(a.sin + (size_t)sp.pos * half) + 16 * lane,
                reinterpret_cast<uint32_t*>(rope + half));
    }

    // the chunk's K and V rows, HBM -> LDS in 16-byte pieces from the 16-byte
    // aligned address at or below the first row (the last piece ends inside
    // the 16-byte granule of the last row's last byte; the row at the step's
    // position is replaced below); they stay in flight while Q is prepared.
    // ncopy counts this wave's copy instructions (lane 0 takes part in every
    // one, so none is skipped).
    const size_t start = (size_t)g * a.head_seq + (size_t)(sp.t0 + jbeg) * hq8;
    const size_t s16 = start & ~(size_t)15;
    const int np = (int)((start + (size_t)cnt * hq8 - s16 + 15) >> 4);
    int ncopy = 0;
    {
        const uint8_t* ks = a.kc + s16;
        const uint8_t* vs = a.vc + s16;
        const int nw = nt >> 6;
        for (int i = w; i * 64 < np; i += nw) {
            if (i * 64 + lane < np) {
                piece16(ks + 16 * (i * 64 + lane), krows + i * 256);
                piece16(vs + 16 * (i * 64 + lane), vrows + i * 256);
            }
            ncopy += 2;
        }
    }
    const uint32_t roff = (uint32_t)(start - s16);   // byte offset of row 0 in krows / vrows
    if (!a.rope) {   // the RoPE factors have landed once at most the row copies are outstanding
        wait_vm_upto(ncopy);
        lds_sync();
    }

    // QK-norm + RoPE + Q8_0 of the group's query heads (and of K, V at pos);
    // LDS-only barriers, so the row copies stay in flight
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
        lds_sync();
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int j = lane + 64 * k;
            if (j < hs) {
                qh[w * hs + j] = nrm[j] * (rq * qh[w * hs + j]);
                if (has_pos && w == 0) kvh[j] = nrm[hs + j] * (rk * kvh[j]);
            }
        }
        lds_sync();
    }
#pragma unroll
    for (int k = 0; k < NR; ++k) {   // RoPE: NEOX (Gemma) or interleaved pairs
        const int p = lane + 64 * k;
        if (p < half) {
            const int i0 = a.neox ? p : 2 * p;
            const int i1 = a.neox ? p + half : 2 * p + 1;
            const float cs = rope[p], sn = rope[half + p];
            const float v0 = qh[w * hs + i0], v1 = qh[w * hs + i1];
            qh[w * hs + i0] = (v0 * cs - v1 * sn) * a.attn_scale;
            qh[w * hs + i1] = (v0 * sn + v1 * cs) * a.attn_scale;
            if (has_pos && w == 0) {
                const float k0 = kvh[i0], k1 = kvh[i1];
                kvh[i0] = k0 * cs - k1 * sn;
                kvh[i1] = k0 * sn + k1 * cs;
            }
        }
    }
    lds_sync();
    // Q8_0 of the head's q, one value per lane (c:3311-3312); all lanes take part
    {
        float v[NQ];
        int8_t q8[NQ];
        uint32_t dh[NQ];
#pragma unroll
        for (int k = 0; k < NQ; ++k) v[k] = lane + 64 * k < hs ? qh[w * hs + lane + 64 * k] : 0.0f;
        quant_lanes<NQ>(v, q8, dh);
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int j = lane + 64 * k;
            if (j < hs) {
                qq[w * hs + j] = q8[k];
                if ((lane & 31) == 0) qd[w * 8 + (j >> 5)] = h2f_exact(dh[k]);
            }
        }
    }
    // K (wave 0) and V (wave 1, or 0 for one-wave groups) of the step, quantized
    // here one value per lane; the copy replaces the copied row in LDS and goes
    // to the cache at the end of the kernel (c:3301-3308)
    const int kvsel = w == 0 ? 0 : (w == 1 ? 1 : -1);
    const bool kv_wave = has_pos && (kvsel >= 0 || km == 1);
    uint32_t kvq[2][NQ], kvdh[2][NQ];
    if (kv_wave) {
#pragma unroll
        for (int sel = 0; sel < 2; ++sel) {
            if (km > 1 && sel != kvsel) continue;
            float v[NQ];
            int8_t q8[NQ];
            uint32_t dh[NQ];
#pragma unroll
            for (int k = 0; k < NQ; ++k) v[k] = lane + 64 * k < hs ? kvh[sel * hs + lane + 64 * k] : 0.0f;
            quant_lanes<NQ>(v, q8, dh);
#pragma unroll
            for (int k = 0; k < NQ; ++k) {
                kvq[sel][k] = (uint8_t)q8[k];
                kvdh[sel][k] = dh[k];
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0): this wave's row copies have landed
    __syncthreads();
    if (kv_wave) {   // the step's own K/V row replaces the copied one
#pragma unroll
        for (int sel = 0; sel < 2; ++sel) {
            if (km > 1 && sel != kvsel) continue;
            uint8_t* rb = reinterpret_cast<uint8_t*>(sel ? vrows : krows) + roff + (size_t)(cnt - 1) * hq8;
#pragma unroll
            for (int k = 0; k < NQ; ++k) {
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

    // scores of head h: lane = position (all of a row's blocks read first)
    const int* qw = reinterpret_cast<const int*>(qq + w * hs);
    const uint8_t* vbytes = reinterpret_cast<const uint8_t*>(vrows) + roff;
    float* fw = f + (size_t)w * 8 * TC;
    constexpr bool kSplit = TC == 32 && NB % 2 == 0;   // two lanes per position
    float sc = -INFINITY;
    if constexpr (kSplit) {
        // lane p sums the first NB/2 block terms of position p, lane p + 32
        // continues that sum over the rest: the reference's order, bit-exact
        constexpr int HB = NB / 2;
        const int pl = lane & 31, hb = (lane >> 5) * HB;
        float t[HB];
        if (pl < cnt) {
            uint32_t kq[HB][8];
            float db[HB];
#pragma unroll
            for (int i = 0; i < HB; ++i) db[i] = row_block(krows, roff + (uint32_t)pl * hq8 + 34u * (hb + i), kq[i]);
#pragma unroll
            for (int i = 0; i < HB; ++i) {
                int isum = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) isum = __builtin_amdgcn_sdot4(qw[8 * (hb + i) + k], (int)kq[i][k], isum, false);
                t[i] = qd[w * 8 + hb + i] * db[i] * (float)isum;
            }
        } else {
#pragma unroll
            for (int i = 0; i < HB; ++i) t[i] = 0.0f;
        }
        float lo = 0.0f;
#pragma unroll
        for (int i = 0; i < HB; ++i) lo += t[i];
        float sum = lane_partner<32>(lo);   // upper lanes: the lower half's sum of the same position
#pragma unroll
        for (int i = 0; i < HB; ++i) sum += t[i];
        const float up = lane_partner<32>(pl < cnt ? cap_score(sum, a.softcap) : -INFINITY);
        if (lane < 32) sc = up;
    } else {
        if (lane < cnt) {
            uint32_t kq[NB][8];
            float db[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) db[b] = row_block(krows, roff + (uint32_t)lane * hq8 + 34u * b, kq[b]);
            float sum = 0.0f;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                int isum = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) isum = __builtin_amdgcn_sdot4(qw[8 * b + k], (int)kq[b][k], isum, false);
                sum += qd[w * 8 + b] * db[b] * (float)isum;
            }
            sc = cap_score(sum, a.softcap);
        }
    }
    const float m = wave_max(sc);
    const float e = lane < cnt ? expf(sc - m) : 0.0f;
    const float l = wave_sum(e);

    // f[b][j] = d(V row j, block b) * e_j, 0 for skipped positions (two
    // lanes per position, as for the scores, when they split them)
    {
        constexpr int FB = kSplit ? NB / 2 : NB;
        const int pl = kSplit ? (lane & 31) : lane;
        const int fb0 = kSplit ? (lane >> 5) * FB : 0;
        const float ep = kSplit ? lane_partner<32>(e) : e;   // upper lanes: their position's e
        const float ej = (kSplit && lane >= 32) ? ep : e;
        if (pl < cnt) {
            const bool skip = ej < 1e-8f;
            uint32_t dv[FB];
#pragma unroll
            for (int i = 0; i < FB; ++i)
                dv[i] = *reinterpret_cast<const uint16_t*>(vbytes + (size_t)pl * hq8 + 34 * (fb0 + i));
#pragma unroll
            for (int i = 0; i < FB; ++i) fw[(fb0 + i) * TC + pl] = skip ? 0.0f : h2f(dv[i]) * ej;
        }
    }
    __syncthreads();
    // V: acc_i += q_ji * f_j over the chunk's rows, eight rows' loads at a time
    const int i0 = lane * PER;
    const bool act = i0 < hs;
    const int b = act ? i0 >> 5 : 0;
    const uint8_t* qrow = vbytes + 34 * b + 2 + (i0 & 31);
    const float* fb = fw + b * TC;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (act) {
        int j = 0;
        for (; j + 8 <= cnt; j += 8) {
            uint32_t qv[8];
            float fv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                qv[u] = v_quants<PER>(qrow + (size_t)(j + u) * hq8);
                fv[u] = fb[j + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int e2 = 0; e2 < PER; ++e2) acc[e2] = fmaf((float)(int8_t)((qv[u] >> (8 * e2)) & 0xffu), fv[u], acc[e2]);
        }
        for (; j < cnt; ++j) {
            const uint32_t q = v_quants<PER>(qrow + (size_t)j * hq8);
#pragma unroll
            for (int e2 = 0; e2 < PER; ++e2) acc[e2] = fmaf((float)(int8_t)((q >> (8 * e2)) & 0xffu), fb[j], acc[e2]);
        }
    }
    float* dst = a.part + ((size_t)h * a.part_chunks + c) * attn_part_row(hs);
    if (act)
#pragma unroll
        for (int e2 = 0; e2 < PER; ++e2) dst[i0 + e2] = acc[e2];
    if (lane == 0) {
        dst[hs] = m;
        dst[hs + 1] = l;
    }
    if (kv_wave) {   // K and V of the step into the cache (c:3301-3308)
#pragma unroll
        for (int sel = 0; sel < 2; ++sel) {
            if (km > 1 && sel != kvsel) continue;
            uint8_t* cd = (sel ? a.vc : a.kc) + (size_t)g * a.head_seq + (size_t)sp.pos * hq8;
#pragma unroll
            for (int k = 0; k < NQ; ++k) {
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
// One round trip for up to 64 chunks (4096 positions): every load is issued
// before anything waits; the first wave holds the chunk maxima and sums
// (lane = chunk, with a running rescale for more than 64 chunks), each thread
// its output's chunk partials, and the weights expf(m_c - M) / S go through
// LDS.  (Reading all chunk slots before the step record arrives was measured
// slower: the extra loads cost more than the wait they save.)
// VPL consecutive floats at p (4, 2 or 1; p aligned to 4 * VPL bytes)
template <int VPL>
__device__ __forceinline__ void load_vec(const float* p, float (&v)[VPL]) {
    if constexpr (VPL == 4) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    } else if constexpr (VPL == 2) {
        const float2 t = *reinterpret_cast<const float2*>(p);
        v[0] = t.x;
        v[1] = t.y;
    } else {
        v[0] = *p;
    }
}

// K chunks' partials of the lane's outputs (pb: the first chunk's, PS floats
// apart), loaded together with no branch (past the nb chunks of the batch
// the last one is read again), then tot += partial * weight for the nb
// chunks in order, chunk b0 + k's weight taken from lane b0 + k of wl.
template <int K, int VPL, int PS>
__device__ __forceinline__ void merge_batch(const float* pb, int nb, float wl, int b0, float (&tot)[VPL]) {
    float pv[K][VPL];
#pragma unroll
    for (int k = 0; k < K; ++k) load_vec<VPL>(pb + (size_t)min(k, nb - 1) * PS, pv[k]);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        if (k < nb) {
            const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), b0 + k));
#pragma unroll
            for (int e = 0; e < VPL; ++e) tot[e] += pv[k][e] * wk;
        }
    }
}

// One wave per head of hs = 32 NB: lane l owns outputs [VPL l, VPL l + VPL)
// (VPL = 4, 2 or 1 for hs up to 256, 128, 64) and reads them from every
// chunk's partial with one vector load, up to 32 chunks' loads issued
// together.  Lane c < 64 first folds the statistics of chunks c, c + 64, ...
// (running max and rescaled sum), then M and S are the wave's max and sum;
// chunk c's weight expf(m_c - M) / S comes from its lane, and each output
// sums its chunks' terms in chunk order.
template <int NB>
__global__ void __launch_bounds__(64) attn_merge_kernel(AttnCArgs a0) {
    constexpr int hs = 32 * NB, ps = attn_part_row(hs);
    constexpr int VPL = NB <= 2 ? 1 : (NB <= 4 ? 2 : 4);
    const AttnCArgs a = token_args(a0, blockIdx.y);
    const Span sp = span_of(a.step, a.window, a.tc);
    const int h = blockIdx.x, nch = sp.n_chunks, lane = threadIdx.x;
    const float* part = a.part + (size_t)h * a.part_chunks * ps;
    // lanes past the row read the last outputs and drop them
    const float* mine = part + min(VPL * lane, hs - VPL);
    float mx = -INFINITY, ssum = 0.0f, m0 = -INFINITY;
    for (int c = lane; c < nch; c += 64) {
        const float2 st = *reinterpret_cast<const float2*>(part + (size_t)c * ps + hs);
        if (c == lane) m0 = st.x;
        const float mn = fmaxf(mx, st.x);
        ssum = ssum * expf(mx - mn) + st.y * expf(st.x - mn);
        mx = mn;
    }
    const float M = wave_max(mx);
    const float S = wave_sum(lane < nch ? ssum * expf(mx - M) : 0.0f);
    float tot[VPL];
#pragma unroll
    for (int e = 0; e < VPL; ++e) tot[e] = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 64) {   // 64 chunks per round
        const int nc = min(64, nch - c0);
        const float mc = c0 == 0 ? m0 : (lane < nc ? part[(size_t)(c0 + lane) * ps + hs] : -INFINITY);
        const float wl = lane < nc ? expf(mc - M) * (1.0f / S) : 0.0f;
        for (int b0 = 0; b0 < nc; b0 += 32) {
            const float* pb = mine + (size_t)(c0 + b0) * ps;
            const int nb = min(32, nc - b0);
            if (nb <= 8) merge_batch<8, VPL, ps>(pb, nb, wl, b0, tot);
            else if (nb <= 16) merge_batch<16, VPL, ps>(pb, nb, wl, b0, tot);
            else if (nb <= 24) merge_batch<24, VPL, ps>(pb, nb, wl, b0, tot);
            else merge_batch<32, VPL, ps>(pb, nb, wl, b0, tot);
        }
    }
    if (VPL * lane < hs) {
#pragma unroll
        for (int e = 0; e < VPL; ++e) a.out[(size_t)h * hs + VPL * lane + e] = tot[e];
    }
}

// ---------------------------------------------------------------------------
// Attention of a prompt batch (c:3232-3359 for each token), FlashAttention
// style: workgroup = one KV group x kPT consecutive tokens of the batch, one
// wave per query head of the group.  The tokens' K/V rows are already in the
// cache (kv_rows_kernel).  Each token's Q row goes through attn_chunk_kernel's
// arithmetic (QK-norm, RoPE with attn_scale, Q8_0), so its Q8_0 row is the
// same; the workgroup then walks the positions its tokens attend to in steps
// of kPP:
//   * the step's K and V rows go HBM -> LDS; K is repacked into int8 rows and
//     fp32 block scales, V dequantized exactly to fp32 and transposed;
//   * scores S^T[pos][tok] per 32-element block on the int8 matrix cores
//     (v_mfma_i32_16x16x32_i8: one instruction is one exact Q8_0 block dot),
//     combined in fp32 in block order as dot_q8_0_q8_0_cache (c:1574-1597):
//     s += (dq * dk) * isum;
//   * a running softmax per token (max m, sum l, earlier terms rescaled by
//     expf(m_old - m)); a position adds to V only when e = expf(s - m) >=
//     1e-8, as in attn_chunk_kernel (e >= the final weight, so every
//     position skipped here is one the reference skips, c:1602);
//   * O^T[d][tok] += V^T[d][pos] e[pos][tok] on the fp32 matrix cores.
// The output is O / l.  Lane l of a wave holds token l % 16 throughout (the
// C layout of a 16 x 16 tile: rows 4(l / 16) .. +3, column l % 16).
// ---------------------------------------------------------------------------
constexpr int kPT = 16;         // tokens per workgroup
constexpr int kPP = 64;         // positions per step
constexpr int kPV = kPP + 4;    // bytes per transposed V row in LDS

typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int prefill_raw_dwords(int hq8) { return chunk_rows_dw(kPP, hq8); }

// LDS bytes of attn_prefill_kernel
__host__ __device__ constexpr size_t prefill_attn_lds(int nb, int km) {
    return (size_t)nb * kPP * 4 * 2 + (size_t)km * kPT * nb * 4 + (size_t)km * 32 * nb * 4 + 2 * kPT * 4 +
           (size_t)32 * nb * kPV + (size_t)kPP * 32 * nb + (size_t)km * kPT * 32 * nb +
           4 * (size_t)prefill_raw_dwords(34 * nb) * 4;
}

// WPH waves per query head: with 2, each takes two of a step's four 16-position
// subtiles with its own running softmax, and the two states are merged at the
// end (the second one through LDS).
template <int NB, int WPH>
__global__ void __launch_bounds__(1024) attn_prefill_kernel(AttnCArgs a0, int ntok) {
    static_assert(WPH == 1 || WPH == 2, "waves per head");
    constexpr int hs = 32 * NB, half = hs / 2, hq8 = 34 * NB, ND = 2 * NB;   // ND: 16-wide d tiles
    constexpr int SPW = 4 / WPH;                                             // subtiles per wave
    extern __shared__ __align__(16) float psm[];
    const int g = blockIdx.x, z0 = blockIdx.y * kPT;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nt = blockDim.x, nw = nt >> 6;
    const int hw = w / WPH, pt = w % WPH;   // head in the group, part
    const int km = a0.kv_mul, h = g * km + hw;
    const bool qwave = pt == 0;              // forms the head's Q rows
    const int rawdw = prefill_raw_dwords(hq8);
    float* kd = psm;                                        // [kPP][NB] K block scales of the step
    float* dvt = kd + kPP * NB;                             // [NB][kPP] V block scales
    float* qd = dvt + kPP * NB;                             // [km][kPT][NB] Q block scales
    float* stg = qd + km * kPT * NB;                        // [km][hs] one Q row being prepared
    int* tpos = reinterpret_cast<int*>(stg + km * hs);      // [kPT] token positions (-1 past the batch)
    int* tbeg = tpos + kPT;                                 // [kPT] first position each token attends to
    int8_t* vqt = reinterpret_cast<int8_t*>(tbeg + kPT);    // [hs][kPV] V quants, transposed
    int8_t* kq = vqt + hs * kPV;                            // [kPP][hs] K quants of the step
    int8_t* qq = kq + kPP * hs;                             // [km][kPT][hs] Q quants
    uint32_t* raw = reinterpret_cast<uint32_t*>(qq + km * kPT * hs);   // [2 buffers][K, V] rows as copied

    if (threadIdx.x < kPT) {
        const int z = z0 + threadIdx.x;
        int p = -1, b = 0;
        if (z < ntok) {
            p = a0.step[2 * z + 1];
            b = a0.window > 0 ? max(0, p - a0.window + 1) : 0;   // c:3316-3321
        }
        tpos[threadIdx.x] = p;
        tbeg[threadIdx.x] = b;
    }

    // ---- Q rows of the tile's tokens for head h (attn_chunk_kernel's arithmetic)
    float* row = stg + hw * hs;
    for (int tt = 0; tt < kPT; ++tt) {
        const int z = z0 + tt;
        int8_t* qrow = qq + (hw * kPT + tt) * hs;
        float* qsc = qd + (hw * kPT + tt) * NB;
        if (z >= ntok) {   // uniform over the workgroup
            if (qwave) {
                for (int j = lane; j < hs; j += 64) qrow[j] = 0;
                if (lane < NB) qsc[lane] = 0.0f;
            }
            continue;
        }
        const AttnCArgs a = token_args(a0, z);
        const int pos = a.step[1];
        float qn[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = lane + 64 * k;
            if (qwave && j < hs) row[j] = a.q[(size_t)h * hs + j];
            qn[k] = (a.q_norm && j < hs) ? a.q_norm[j] : 0.0f;
        }
        __syncthreads();
        if (a.q_norm) {   // per-head rmsnorm (c:3151-3165)
            float rq = 0.0f;
            if (qwave) {
                float ssq = 0.0f;
                for (int j = lane; j < hs; j += 64) ssq += row[j] * row[j];
                ssq = wave_sum(ssq);
                rq = 1.0f / sqrtf(ssq * a.inv_hs + a.eps);
            }
            __syncthreads();
            if (qwave) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int j = lane + 64 * k;
                    if (j < hs) row[j] = qn[k] * (rq * row[j]);
                }
            }
            __syncthreads();
        }
        const float* cosr = a.cos + (size_t)pos * half;
        const float* sinr = a.sin + (size_t)pos * half;
#pragma unroll
        for (int k = 0; k < 2; ++k) {   // RoPE with the attention scale (c:3240-3296)
            const int p = lane + 64 * k;
            if (qwave && p < half) {
                const int i0 = a.neox ? p : 2 * p;
                const int i1 = a.neox ? p + half : 2 * p + 1;
                const float v0 = row[i0], v1 = row[i1], cs = cosr[p], sn = sinr[p];
                row[i0] = (v0 * cs - v1 * sn) * a.attn_scale;
                row[i1] = (v0 * sn + v1 * cs) * a.attn_scale;
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; ++k) {   // Q8_0 of q (c:3311-3312), one value per lane
            const int j = lane + 64 * k;
            if (qwave && k * 64 < hs) {
                uint32_t dh;
                const int8_t q8 = quant_lane(j < hs ? row[j] : 0.0f, dh);   // all lanes take part
                if (j < hs) {
                    qrow[j] = q8;
                    if ((lane & 31) == 0) qsc[j >> 5] = h2f_exact(dh);
                }
            }
        }
        __syncthreads();
    }

    __syncthreads();
    // ---- positions the tile attends to
    int lo = 0x7fffffff, hi = -1;
    for (int tt = 0; tt < kPT; ++tt) {
        if (tpos[tt] >= 0) {
            lo = min(lo, tbeg[tt]);
            hi = max(hi, tpos[tt]);
        }
    }
    const int tok = lane & 15, gq = lane >> 4;
    const int my_pos = tpos[tok], my_beg = tbeg[tok];
    const int8_t* qrow = qq + (hw * kPT + tok) * hs;
    const float* qsc = qd + (hw * kPT + tok) * NB;
    float m_run = -INFINITY, l_run = 0.0f;
    floatx4 acc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) acc[d] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const size_t head_base = (size_t)g * a0.head_seq;

    // the K and V rows of the step at p0 into raw buffer `buf`: 16-byte
    // pieces from the 16-byte aligned address at or below the first row (the
    // copies of the next step are in flight while this step is computed)
    const int p_first = hi < 0 ? 0 : (lo & ~(kPP - 1));
    auto copy_rows = [&](int p0, int buf) {
        const int cnt = min(kPP, hi + 1 - p0);
        const size_t start = head_base + (size_t)p0 * hq8;
        const size_t s16 = start & ~(size_t)15;
        const int np = (int)((start + (size_t)cnt * hq8 - s16 + 15) >> 4);
        uint32_t* kr = raw + (size_t)buf * 2 * rawdw;
        for (int i = w; i * 64 < np; i += nw) {
            if (i * 64 + lane < np) {
                piece16(a0.kc + s16 + 16 * (i * 64 + lane), kr + i * 256);
                piece16(a0.vc + s16 + 16 * (i * 64 + lane), kr + rawdw + i * 256);
            }
        }
    };
    if (hi >= 0) copy_rows(p_first, 0);
    int buf = 0;
    for (int p0 = p_first; p0 <= hi; p0 += kPP, buf ^= 1) {
        const int cnt = min(kPP, hi + 1 - p0);   // rows p0 .. p0 + cnt - 1
        const uint32_t roff = (uint32_t)((head_base + (size_t)p0 * hq8) & 15);
        const uint32_t* kraw = raw + (size_t)buf * 2 * rawdw;
        const uint32_t* vraw = kraw + rawdw;
        __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0): this wave's copies have landed
        __syncthreads();   // every wave's copies landed; the previous step's LDS reads are done
        // repack: K block (p, b) -> int8 row + scale, V block -> int8 V^T + scale
        for (int task = threadIdx.x; task < kPP * NB; task += nt) {
            const int p = task % kPP, b = task / kPP;
            uint32_t kqw[8], vqw[8];
            float dk = 0.0f, dv = 0.0f;
            if (p < cnt) {
                dk = row_block(kraw, roff + (uint32_t)(p * hq8 + 34 * b), kqw);
                dv = row_block(vraw, roff + (uint32_t)(p * hq8 + 34 * b), vqw);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) kqw[e] = vqw[e] = 0u;
            }
            kd[p * NB + b] = dk;
            dvt[b * kPP + p] = dv;
            uint4* kdst = reinterpret_cast<uint4*>(kq + p * hs + 32 * b);
            kdst[0] = make_uint4(kqw[0], kqw[1], kqw[2], kqw[3]);
            kdst[1] = make_uint4(kqw[4], kqw[5], kqw[6], kqw[7]);
#pragma unroll
            for (int e = 0; e < 32; ++e) vqt[(32 * b + e) * kPV + p] = (int8_t)((vqw[e >> 2] >> (8 * (e & 3))) & 0xffu);
        }
        __syncthreads();
        // the next step's rows go into the other buffer while this one is used
        if (p0 + kPP <= hi) copy_rows(p0 + kPP, buf ^ 1);

        // scores of head h over this wave's subtiles: S^T[pos][tok], pos =
        // st * 16 + 4 gq + r, tok = lane % 16
        float sc[SPW][4];
#pragma unroll
        for (int s2 = 0; s2 < SPW; ++s2) {
            const int st = pt * SPW + s2;
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[s2][r] = 0.0f;
            const int8_t* krow = kq + (st * 16 + tok) * hs + 8 * gq;   // A: position row lane % 16
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const long av = *reinterpret_cast<const long*>(krow + 32 * b);
                const long bv = *reinterpret_cast<const long*>(qrow + 32 * b + 8 * gq);
                const int32x4 is = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, int32x4{0, 0, 0, 0}, 0, 0, 0);
                const float qs = qsc[b];
#pragma unroll
                for (int r = 0; r < 4; ++r) sc[s2][r] += qs * kd[(st * 16 + 4 * gq + r) * NB + b] * (float)is[r];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int pa = p0 + st * 16 + 4 * gq + r;
                sc[s2][r] = cap_score(sc[s2][r], a0.softcap);
                if (my_pos < 0 || pa > my_pos || pa < my_beg) sc[s2][r] = -INFINITY;
            }
        }
        // running softmax of token tok (its positions sit in lanes tok + 16 j)
        float cm = -INFINITY;
#pragma unroll
        for (int s2 = 0; s2 < SPW; ++s2)
#pragma unroll
            for (int r = 0; r < 4; ++r) cm = fmaxf(cm, sc[s2][r]);
        cm = fmaxf(cm, lane_partner<16>(cm));
        cm = fmaxf(cm, lane_partner<32>(cm));
        const float mn = fmaxf(m_run, cm);
        const bool none = mn == -INFINITY;   // nothing attended yet
        const float alpha = none ? 1.0f : expf(m_run - mn);
        float f[SPW][4], ls = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < SPW; ++s2)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = sc[s2][r] == -INFINITY ? 0.0f : expf(sc[s2][r] - mn);
                ls += e;
                f[s2][r] = e < 1e-8f ? 0.0f : e;
            }
        ls += lane_partner<16>(ls);
        ls += lane_partner<32>(ls);
        l_run = l_run * alpha + ls;
        m_run = mn;
        // O^T[d][tok] = alpha O^T + V^T[d][pos] f[pos][tok], V^T expanded
        // exactly (q * d) right before its matrix instruction
#pragma unroll
        for (int d = 0; d < ND; ++d) {
            acc[d] *= alpha;
            const int8_t* vrow = vqt + (d * 16 + tok) * kPV + 4 * gq;   // A: V^T row d, positions 4 gq ..
            const float* dvr = dvt + (d >> 1) * kPP + 4 * gq;            // block d * 16 / 32 of those positions
#pragma unroll
            for (int s2 = 0; s2 < SPW; ++s2) {
                const int st = pt * SPW + s2;
                const uint32_t q4 = *reinterpret_cast<const uint32_t*>(vrow + st * 16);
                const float4 d4 = *reinterpret_cast<const float4*>(dvr + st * 16);
                acc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int8_t)(q4 & 0xffu) * d4.x, f[s2][0], acc[d], 0, 0, 0);
                acc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int8_t)((q4 >> 8) & 0xffu) * d4.y, f[s2][1], acc[d], 0,
                                                              0, 0);
                acc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int8_t)((q4 >> 16) & 0xffu) * d4.z, f[s2][2], acc[d], 0,
                                                              0, 0);
                acc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int8_t)(q4 >> 24) * d4.w, f[s2][3], acc[d], 0, 0, 0);
            }
        }
    }
    if constexpr (WPH == 2) {
        // the second part's (m, l, O) through LDS (the copy buffers are free:
        // no copy is in flight after the last step), merged into the first's
        __syncthreads();
        float* mg = reinterpret_cast<float*>(raw) + (size_t)(hw * 64 + lane) * (2 + 4 * ND);
        if (pt == 1) {
            mg[0] = m_run;
            mg[1] = l_run;
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 4; ++r) mg[2 + 4 * d + r] = acc[d][r];
        }
        __syncthreads();
        if (pt == 0) {
            const float m1 = mg[0], l1 = mg[1];
            const float M = fmaxf(m_run, m1);
            const float s0 = m_run == -INFINITY ? 0.0f : expf(m_run - M);
            const float s1 = m1 == -INFINITY ? 0.0f : expf(m1 - M);
            l_run = l_run * s0 + l1 * s1;
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[d][r] = acc[d][r] * s0 + mg[2 + 4 * d + r] * s1;
        }
    }
    // out[tok][h][d] = O / l: lane holds d = 16 dt + 4 gq .. + 3 of token tok
    const int z = z0 + tok;
    if (pt == 0 && z < ntok && my_pos >= 0) {
        const float inv = 1.0f / l_run;
        float* o = a0.out + (size_t)z * a0.out_stride + (size_t)h * hs + 4 * gq;
#pragma unroll
        for (int d = 0; d < ND; ++d)
            *reinterpret_cast<float4*>(o + d * 16) = make_float4(acc[d][0] * inv, acc[d][1] * inv, acc[d][2] * inv,
                                                                 acc[d][3] * inv);
    }
}

// ---------------------------------------------------------------------------
// Attention of one decode step (c:3232-3359) with one workgroup per query
// head (any context; the faster choice for short ones).  The position loop is split
// over kHW waves: wave w takes chunks w, w + kHW, ... of cp positions and
// streams each chunk's K rows and V rows HBM -> LDS (dwordx4 copies into two
// slots of its own: the V rows land while the scores are formed, the next K
// rows while V is accumulated).  Per chunk, as in attn_chunk_kernel: the
// exact Q8_0 score of each position (lane = position), e = expf(s - m) with
// m the wave's running maximum (earlier chunks rescaled by expf(m_old - m)),
// and the unnormalized V accumulation sum_t q_t * (d_t * e_t), a position
// skipped when e < 1e-8.  The waves' (m, l, acc) are merged at the end into
// sum_w acc_w * expf(m_w - M) / S.
//   The step's own K and V rows (QK-norm, RoPE, Q8_0, the arithmetic of
// attn_chunk_kernel) are formed by every workgroup of the KV group, used
// from LDS, and written to the cache by the group's first head.
// blockIdx.x = head-in-group * n_kv + group: with n_kv a multiple of 8 the
// heads of a group run on one XCD and share its L2.
// ---------------------------------------------------------------------------
constexpr int kHW = 16;                           // waves per workgroup
constexpr int kHCopies = 4;                       // dwordx4 copy instructions per slot
constexpr int kHSlot = kHCopies * 1024;           // bytes per K or V slot
constexpr int kHRows = kHSlot - 16;               // bytes of rows per chunk (room for 15 B of alignment slack)

__host__ __device__ constexpr int head_chunk_positions(int hq8) { return kHRows / hq8 < 64 ? kHRows / hq8 : 64; }

// vmcnt(N) (expcnt and lgkmcnt not waited for)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// cnt rows of one KV head's cache into an LDS slot, from the 16-byte aligned
// address at or below the first row: kHCopies instructions, lane l of
// instruction i copying 16-byte piece 64 i + l (pieces past the rows repeat
// the last one).  Every lane of every instruction copies, so the code has no
// branch and the waits that follow can count the copies.  Returns the first
// row's offset in the slot.
__device__ __forceinline__ uint32_t head_copy(uint32_t* slot, const uint8_t* rows, int cnt, int hq8, int lane) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(rows);
    const uint8_t* a16 = reinterpret_cast<const uint8_t*>(a & ~(uintptr_t)15);
    const uint32_t roff = (uint32_t)(a & 15);
    const int np = (int)((roff + (uint32_t)cnt * hq8 + 15) >> 4);   // pieces, <= kHSlot / 16 (cnt * hq8 <= kHRows)
    __builtin_amdgcn_s_waitcnt(0xc07f);                             // lgkmcnt(0): earlier reads of the slot done
#pragma unroll
    for (int i = 0; i < kHCopies; ++i) {
        const int pc = min(64 * i + lane, np - 1);
        __builtin_amdgcn_global_load_lds(a16 + 16 * pc, (lds_void*)(slot + 256 * i), 16, 0, 0);
    }
    return roff;
}

template <int NB>
__global__ void __launch_bounds__(1024) attn_head_kernel(AttnCArgs a) {
    constexpr int hs = 32 * NB, nb = NB, half = hs / 2;
    constexpr int PER = NB <= 2 ? 1 : (NB <= 4 ? 2 : 4);   // V outputs per lane, inside one 32-block
    extern __shared__ __align__(16) uint32_t hl[];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hq8 = 34 * NB;
    const int n_kv = a.n_heads / a.kv_mul;
    const int g = blockIdx.x % n_kv, hg = blockIdx.x / n_kv, h = g * a.kv_mul + hg;
    const Span sp = span_of(a.step, a.window, a.tc);
    const int cp = head_chunk_positions(hq8);
    const int nch = (sp.na + cp - 1) / cp;
    const int nk = w < nch ? (nch - 1 - w) / kHW + 1 : 0;   // chunks of this wave

    // LDS: [kHW][K slot, V slot], [kHW][hs + 2] wave results (the prologue's
    // staging rows alias them), hs int8 q, 8 q scales, the step's K and V rows
    uint32_t* kslot = hl + (size_t)w * 2 * (kHSlot / 4);
    uint32_t* vslot = kslot + kHSlot / 4;
    float* red = reinterpret_cast<float*>(hl + (size_t)kHW * 2 * (kHSlot / 4));
    int8_t* qq = reinterpret_cast<int8_t*>(red + kHW * (hs + 2));
    float* qd = reinterpret_cast<float*>(qq + 256);
    uint8_t* kvrow = reinterpret_cast<uint8_t*>(qd + 8);   // [2][hq8 rounded up to 4]
    const int rowst = (hq8 + 3) & ~3;

    // ---- the step's rows (wave 0: q of head h, the RoPE row and q_norm;
    // 1: k of group g and k_norm; 2: v) and this wave's first K and V rows,
    // all as LDS copies: explicit waits count them, so waiting for the step's
    // rows never waits for the cache rows
    const int role = w < 3 ? w : -1;
    float* stg = red;   // [q, q_norm, k, k_norm, v][hs], cos, sin [half]: aliases the wave results
    auto copy_vec = [&](float* dst, const float* src, int n) {   // n floats, dword pieces
        for (int i = 0; 64 * i < n; ++i)
            if (64 * i + lane < n) __builtin_amdgcn_global_load_lds(src + 64 * i + lane, (lds_void*)(dst + 64 * i), 4, 0, 0);
    };
    if (role == 0) {
        copy_vec(stg, a.q + (size_t)h * hs, hs);
        if (a.q_norm) copy_vec(stg + hs, a.q_norm, hs);
        copy_vec(stg + 5 * hs, a.cos + (size_t)sp.pos * half, half);
        copy_vec(stg + 5 * hs + half, a.sin + (size_t)sp.pos * half, half);
    } else if (role == 1) {
        copy_vec(stg + 2 * hs, a.k + (size_t)g * hs, hs);
        if (a.k_norm) copy_vec(stg + 3 * hs, a.k_norm, hs);
    } else if (role == 2) {
        copy_vec(stg + 4 * hs, a.v + (size_t)g * hs, hs);
    }
    const size_t head_base = (size_t)g * a.head_seq;
    auto chunk_rows = [&](int c, int& cnt) {
        const int j0 = c * cp;
        cnt = min(cp, sp.na - j0);
        return head_base + (size_t)(sp.t0 + j0) * hq8;
    };
    uint32_t roff;
    {   // waves past the last chunk copy it too (unused), so the copies are unconditional
        int cnt;
        const size_t off = chunk_rows(min(w, nch - 1), cnt);
        roff = head_copy(kslot, a.kc + off, cnt, hq8, lane);
        head_copy(vslot, a.vc + off, cnt, hq8, lane);
    }
    wait_vm<2 * kHCopies>();   // the step's rows have landed
    lds_sync();

    // ---- QK-norm (c:3151-3165), RoPE (c:3240-3296) and Q8_0 of q (c:3311-3312),
    // k and v (c:3301-3308), with the arithmetic of attn_chunk_kernel
    if (role == 0 || role == 1) {
        float* row = stg + 2 * role * hs;
        const bool normed = role == 0 ? a.q_norm != nullptr : a.k_norm != nullptr;
        if (normed) {
            float xv[4];
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int j = lane + 64 * k;
                xv[k] = j < hs ? row[j] : 0.0f;
                ss += xv[k] * xv[k];
            }
            ss = wave_sum(ss);
            const float r = 1.0f / sqrtf(ss * a.inv_hs + a.eps);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int j = lane + 64 * k;
                if (j < hs) row[j] = row[hs + j] * (r * xv[k]);
            }
        }
    }
    lds_sync();
    if (role == 0 || role == 1) {
        float* row = stg + 2 * role * hs;
        const float* cosr = stg + 5 * hs;
        const float* sinr = cosr + half;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int p = lane + 64 * k;
            if (p < half) {
                const int i0 = a.neox ? p : 2 * p;
                const int i1 = a.neox ? p + half : 2 * p + 1;
                const float v0 = row[i0], v1 = row[i1], cs = cosr[p], sn = sinr[p];
                if (role == 0) {
                    row[i0] = (v0 * cs - v1 * sn) * a.attn_scale;
                    row[i1] = (v0 * sn + v1 * cs) * a.attn_scale;
                } else {
                    row[i0] = v0 * cs - v1 * sn;
                    row[i1] = v0 * sn + v1 * cs;
                }
            }
        }
    }
    lds_sync();
    uint32_t kvq[4], kvdh[4];
    if (role >= 0) {
        const float* row = stg + 2 * role * hs;
        uint8_t* rb = kvrow + (role == 2 ? rowst : 0);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = lane + 64 * k;
            if (k * 64 < hs) {
                uint32_t dh;
                const int8_t q8 = quant_lane(j < hs ? row[j] : 0.0f, dh);   // all lanes take part
                kvq[k] = (uint8_t)q8;
                kvdh[k] = dh;
                if (j < hs) {
                    const int b = j >> 5;
                    if (role == 0) {
                        qq[j] = q8;
                        if ((lane & 31) == 0) qd[b] = h2f_exact(dh);
                    } else {
                        rb[34 * b + 2 + (j & 31)] = (uint8_t)q8;
                        if ((lane & 31) == 0) {
                            rb[34 * b] = (uint8_t)(dh & 0xff);
                            rb[34 * b + 1] = (uint8_t)(dh >> 8);
                        }
                    }
                }
            }
        }
    }
    lds_sync();   // q and the step's rows ready; the staging rows are free again

    // ---- this wave's chunks
    const int i0 = lane * PER;
    const bool act = i0 < hs;
    const int vb = act ? i0 >> 5 : 0;
    const uint32_t doff = 34u * vb, qoff = 34u * vb + 2u + (uint32_t)(i0 & 31);
    // q of the head: the same in every lane
    int qw[8 * NB];
    float qs[NB];
#pragma unroll
    for (int i = 0; i < 8 * NB; ++i) qw[i] = __builtin_amdgcn_readfirstlane(reinterpret_cast<const int*>(qq)[i]);
#pragma unroll
    for (int b = 0; b < NB; ++b) qs[b] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(qd[b])));
    float m_run = -INFINITY, l_run = 0.0f;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t* kpos = reinterpret_cast<const uint32_t*>(kvrow);
    const uint8_t* vpos = kvrow + rowst;
    for (int k = 0; k < nk; ++k) {
        const int c = w + k * kHW;
        int cnt;
        (void)chunk_rows(c, cnt);
        const bool last = c == nch - 1;   // holds the step's position, at row cnt - 1
        const uint32_t ro_c = roff;       // this chunk's first-row offset in both slots
        wait_vm<kHCopies>();              // the K rows have landed (the V copy may be in flight)
        float sc = -INFINITY;
        if (lane < cnt) {   // dot_q8_0_q8_0_cache (c:1574-1597): exact block dots in block order
            const bool mine = last && lane == cnt - 1;
            const uint32_t* kb = mine ? kpos : kslot;
            const uint32_t ro = mine ? 0u : ro_c + (uint32_t)lane * hq8;
            uint32_t kq[NB][8];
            float db[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) db[b] = row_block(kb, ro + 34u * b, kq[b]);
            float sum = 0.0f;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                int isum = 0;
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) isum = __builtin_amdgcn_sdot4(qw[8 * b + e2], (int)kq[b][e2], isum, false);
                sum += qs[b] * db[b] * (float)isum;
            }
            sc = cap_score(sum, a.softcap);
        }
        const float mn = fmaxf(m_run, wave_max(sc));
        const float alpha = expf(m_run - mn);   // 0 for the first chunk
        const float e = lane < cnt ? expf(sc - mn) : 0.0f;
        l_run = l_run * alpha + wave_sum(e);
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) acc[e2] *= alpha;
        m_run = mn;
        // the next chunk's K rows go into the K slot (its reads are done)
        // while this chunk's V rows are accumulated
        const bool more = k + 1 < nk;
        size_t off2 = 0;
        int cnt2 = 0;
        if (more) {
            off2 = chunk_rows(c + kHW, cnt2);
            roff = head_copy(kslot, a.kc + off2, cnt2, hq8, lane);
            wait_vm<kHCopies>();   // this chunk's V rows have landed
        } else {
            wait_vm<0>();
        }
        if (act) {
            const uint8_t* vrows = reinterpret_cast<const uint8_t*>(vslot) + ro_c;
            const int nrow = last ? cnt - 1 : cnt;   // the step's own row comes from vpos
            int j = 0;
            for (; j + 8 <= nrow; j += 8) {
                uint32_t dv[8], qv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint8_t* row = vrows + (size_t)(j + u) * hq8;
                    dv[u] = *reinterpret_cast<const uint16_t*>(row + doff);
                    qv[u] = v_quants<PER>(row + qoff);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    v_accum<PER>(dv[u], qv[u], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j + u)), acc);
            }
            for (; j < nrow; ++j) {
                const uint8_t* row = vrows + (size_t)j * hq8;
                v_accum<PER>(*reinterpret_cast<const uint16_t*>(row + doff), v_quants<PER>(row + qoff),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j)), acc);
            }
            if (last)
                v_accum<PER>(*reinterpret_cast<const uint16_t*>(vpos + doff), v_quants<PER>(vpos + qoff),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), cnt - 1)), acc);
        }
        if (more) head_copy(vslot, a.vc + off2, cnt2, hq8, lane);
    }
    wait_vm<0>();   // waves without chunks: their unused copies

    // ---- merge the waves: out = sum_w acc_w * expf(m_w - M) / S
    float* rw = red + w * (hs + 2);
    if (act)
        for (int e2 = 0; e2 < PER; ++e2) rw[i0 + e2] = acc[e2];
    if (lane == 0) {
        rw[hs] = m_run;
        rw[hs + 1] = l_run;
    }
    lds_sync();
    if (w == 0) {
        const float mw = lane < kHW ? red[lane * (hs + 2) + hs] : -INFINITY;
        const float lw = lane < kHW ? red[lane * (hs + 2) + hs + 1] : 0.0f;
        const float M = wave_max(mw);
        const float ex = lane < kHW ? expf(mw - M) : 0.0f;   // 0 for waves without chunks
        const float S = wave_sum(lw * ex);
        const float wt = ex * (1.0f / S);
        if (act) {
            float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q = 0; q < kHW; ++q) {
                const float wq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wt), q));
                for (int e2 = 0; e2 < PER; ++e2) o[e2] += red[q * (hs + 2) + i0 + e2] * wq;
            }
            for (int e2 = 0; e2 < PER; ++e2) a.out[(size_t)h * hs + i0 + e2] = o[e2];
        }
    }
    // the step's K and V rows into the cache (c:3301-3308), by the group's first head
    if (hg == 0 && (role == 1 || role == 2)) {
        uint8_t* cd = (role == 2 ? a.vc : a.kc) + head_base + (size_t)sp.pos * hq8;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = lane + 64 * k;
            if (j < hs) {
                const int b = j >> 5;
                cd[34 * b + 2 + (j & 31)] = (uint8_t)kvq[k];
                if ((lane & 31) == 0) {
                    cd[34 * b] = (uint8_t)(kvdh[k] & 0xff);
                    cd[34 * b + 1] = (uint8_t)(kvdh[k] >> 8);
                }
            }
        }
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
// every group of 64 logits (indices >= k); kernel 2 walks the groups in order
// and only visits groups whose maximum beats the current minimum.  Kernel 2
// is one workgroup: waves 1..15 stream the logits and group maxima through
// LDS in blocks of kScanBlock while wave 0, which holds the slots, scans the
// previous block there, so a visited group costs an LDS read rather than a
// dependent global load.  For k <= 64 wave 0 also keeps the slots as a list
// sorted by (value, slot), one entry per lane (NaN sorted as +inf: the
// reference never takes a NaN slot as its minimum): the minimum is lane 0,
// and a replacement drops it and inserts the new (value, slot) at its rank,
// one ballot and a one-lane shift instead of a search over the slots.
constexpr int kSlotsPerLane = 16;            // k <= 1024
constexpr int kScanBlock = 16384;            // logits per LDS block (256 groups)

__global__ void __launch_bounds__(1024) topk_groupmax_kernel(const float* __restrict__ l, int n, int k, int ng,
                                                             float* gmax) {
    const int g = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int i = 64 * g + lane;
    float v = (i >= k && i < n) ? l[i] : -INFINITY;
    v = wave_max(v);
    if (lane == 0 && g < ng) gmax[g] = v;
}

// R: slot rows of 64 in use (k <= 64 R), so the minimum search after each
// replacement only visits live rows
template <int R>
__global__ void __launch_bounds__(1024) topk_scan_kernel(const float* __restrict__ l, int n, int k,
                                                         const float* __restrict__ gmax, int ng, float* out_v,
                                                         int* out_i, HostSlots pub) {
    static_assert(R >= 1 && R <= kSlotsPerLane, "slot rows");
    extern __shared__ __align__(16) float tl[];   // [2][kScanBlock] logits, then [2][256] group maxima
    float* tg = tl + 2 * kScanBlock;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nblk = (n + kScanBlock - 1) / kScanBlock;
    // block b into buffer b & 1 by waves 1..15: 64-float pieces, each lane one
    // dword (indices past the end repeat the last logit or group maximum; the
    // scan masks them by index)
    auto fill = [&](int b) {
        float* dst = tl + (b & 1) * kScanBlock;
        for (int pc = w - 1; pc < kScanBlock / 64; pc += 15) {
            const int i = min(b * kScanBlock + 64 * pc + lane, n - 1);
            __builtin_amdgcn_global_load_lds(l + i, (lds_void*)(dst + 64 * pc), 4, 0, 0);
        }
        if (w <= 4) {
            const int gi = min(b * (kScanBlock / 64) + 64 * (w - 1) + lane, ng - 1);
            __builtin_amdgcn_global_load_lds(gmax + gi, (lds_void*)(tg + (b & 1) * 256 + 64 * (w - 1)), 4, 0, 0);
        }
    };
    if (w > 0) fill(0);
    float sv[R];
    int si[R];
    float cur = 0.0f;
    int cur_slot = 0;
    // The reference's minimum (c:4819-4826, 4835-4842): it starts at slot 0
    // and moves to a slot only on a strictly smaller value, so it is the
    // first slot holding the smallest value, NaN slots never chosen unless
    // slot 0 is NaN (which then stays the minimum).  Lane minima, a register
    // butterfly minimum, then the first slot row whose ballot holds it.
    auto find_min = [&](float& mv, int& ms) {
        float lv = INFINITY;
#pragma unroll
        for (int j = 0; j < R; ++j)
            if (lane + 64 * j < k) lv = fminf(lv, sv[j]);
        float m = -wave_max(-lv);
        int slot = 0;
#pragma unroll
        for (int j = R - 1; j >= 0; --j) {
            if (64 * j < k) {
                const uint64_t hit = __ballot(lane + 64 * j < k && sv[j] == m);
                if (hit) slot = 64 * j + __ffsll((unsigned long long)hit) - 1;
            }
        }
        const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv[0]), 0));
        if (s0 != s0) {
            m = s0;
            slot = 0;
        }
        mv = m;
        ms = slot;
    };
    auto lane_val = [](float v, int j) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j)); };
    // k <= 64: the sorted list (key, ks) by rank; sv[0], si[0] stay the slot
    // values and indices by slot (lane = slot)
    float key = INFINITY;
    int ks = 64 + lane;   // lanes past k: sentinels after every slot
    if (w == 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int s = lane + 64 * j;
            sv[j] = s < k ? l[s] : INFINITY;
            si[j] = s < k ? s : -1;
        }
        if constexpr (R == 1) {
            if (lane < k) {
                key = sv[0] != sv[0] ? INFINITY : sv[0];
                ks = lane;
            }
            // bitonic sort by (key, ks), ascending; the pairs are distinct
            for (int size = 2; size <= 64; size <<= 1) {
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    const float ok = __shfl_xor(key, stride, 64);
                    const int os = __shfl_xor(ks, stride, 64);
                    const bool other_less = ok < key || (ok == key && os < ks);
                    const bool want_min = ((lane & stride) == 0) == ((lane & size) == 0);
                    if (want_min ? other_less : !other_less) {
                        key = ok;
                        ks = os;
                    }
                }
            }
            // a NaN in slot 0 stays the reference's minimum: nothing is ever
            // greater, so nothing is replaced
            const float s0 = lane_val(sv[0], 0);
            cur = s0 != s0 ? s0 : lane_val(key, 0);
        } else {
            find_min(cur, cur_slot);
        }
    }
    // logits[i] = bv > cur replaces the minimum slot
    auto replace = [&](float bv, int i) {
        if constexpr (R == 1) {
            const int sh = __builtin_amdgcn_readlane(ks, 0);   // the minimum's slot
            // bitwise, not short-circuit: no exec-mask branches on this chain
            const bool before = (lane >= 1) & (lane < k) & ((key < bv) | ((key == bv) & (ks < sh)));
            const int r = __popcll(__ballot(before));
            // lane + 1's entry (DPP wave_shl:1; lane 63 keeps its own, never used)
            const float kn = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(key), __float_as_int(key),
                                                                        0x130, 0xF, 0xF, false));
            const int sn = __builtin_amdgcn_update_dpp(ks, ks, 0x130, 0xF, 0xF, false);
            key = lane < r ? kn : (lane == r ? bv : key);
            ks = lane < r ? sn : (lane == r ? sh : ks);
            if (lane == sh) {
                sv[0] = bv;
                si[0] = i;
            }
            cur = lane_val(key, 0);
        } else {
            if (lane == (cur_slot & 63)) {
#pragma unroll
                for (int jj = 0; jj < R; ++jj)
                    if (jj == (cur_slot >> 6)) { sv[jj] = bv; si[jj] = i; }
            }
            find_min(cur, cur_slot);
        }
    };
    wait_vm<0>();
    __syncthreads();
    for (int b = 0; b < nblk; ++b) {
        if (w > 0) {
            if (b + 1 < nblk) fill(b + 1);
        } else {
            const float* lb = tl + (b & 1) * kScanBlock;
            const float* gb = tg + (b & 1) * 256;
            for (int j0 = 0; j0 < kScanBlock / 64; j0 += 64) {
                const int G = b * (kScanBlock / 64) + j0 + lane;
                const float gm = G < ng ? gb[j0 + lane] : -INFINITY;
                uint64_t flagged = __ballot(gm > cur);
                while (flagged) {
                    const int j = __ffsll((unsigned long long)flagged) - 1;
                    flagged &= flagged - 1;
                    if (!(lane_val(gm, j) > cur)) continue;
                    const int gofs = 64 * (j0 + j);
                    const int base = b * kScanBlock + gofs;
                    const int i = base + lane;
                    const float v = (i >= k && i < n) ? lb[gofs + lane] : -INFINITY;
                    // candidates in index order; after each replacement the
                    // mask is narrowed to those still above the new minimum,
                    // so every iteration replaces
                    uint64_t cand = __ballot(v > cur);
                    while (cand) {
                        const int c = __ffsll((unsigned long long)cand) - 1;
                        replace(lane_val(v, c), base + c);
                        cand &= __ballot(v > cur) & ~((2ull << c) - 1ull);
                    }
                }
            }
        }
        wait_vm<0>();      // this wave's copies of block b + 1 have landed
        __syncthreads();   // and every wave's; wave 0 is done with block b
    }
    if (w == 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int s = lane + 64 * j;
            if (s < k) { out_v[s] = sv[j]; out_i[s] = si[j]; }
        }
        if (pub.v) {   // the slots to the host, then the sequence word once they are visible there
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const int s = lane + 64 * j;
                if (s < k) {
                    __hip_atomic_store(pub.v + s, sv[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    __hip_atomic_store(pub.i + s, si[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
            }
            __threadfence_system();
            if (lane == 0) __hip_atomic_store(pub.seq_word, pub.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
void launch_embed_step(const Model& m, int token, int pos, hipStream_t s, const int* dtok, HostToken ht) {
    const RopeRows rope{{m.cos_d, m.sin_d, m.cos_s, m.sin_s}, m.hs / 2, m.rope_cur};
    const bool later = dtok || ht.word;   // the token is read when the kernel runs
    launch_embed_row(m.emb.type, m.emb.w + (later ? 0 : (size_t)token * m.emb.rb), m.emb.cols,
                     m.is_gemma ? m.embed_scale : 0.0f, m.x, token, pos, m.step, &rope, s, dtok, m.emb.rb, ht);
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

void launch_attention(const Model& m, int l, float* out, bool per_head, hipStream_t s) {
    launch_attention(m, l, AttnIO{m.q, m.k, m.v, m.step, out}, per_head, s);
}

// L3P_ATTN_HEAD=1 / 0 forces one attention or the other; by default the
// per-head kernel takes steps attending to fewer positions than
// attention_head_limit, where it is the faster of the two on MI355X (its
// time grows with the positions one CU streams, chunks + merge stay near
// 9-11 us): about 450 positions at head_dim 128 (Llama-3-8B's 32/8 heads:
// 7.5 against 9.0 us at 257, 10.1 against 9.6 us at 513) and 190 at
// head_dim 256 (Gemma-2-2B's 8/4 heads: 7.9 against 10.2 us at 65, 11.8
// against 10.4 us at 257).
int attention_head_limit(const Model& m) { return m.hs >= 192 ? 192 : 448; }

bool attention_per_head(const Model& m, int pos) {
    const char* e = getenv("L3P_ATTN_HEAD");
    if (e && *e) return atoi(e) != 0;
    return pos < attention_head_limit(m);
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
    a.rope = m.rope_cur + (use_swa ? m.hs : 0);   // decode steps; prompt batches read the tables
    a.kc = m.kc + (size_t)l * m.layer_kv;
    a.vc = m.vc + (size_t)l * m.layer_kv;
    a.step = io.step;
    a.part = m.part_acc;
    a.part_chunks = m.max_chunks;
    a.tc = kTC;
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
    a.softcap = m.attn_softcap;
    return a;
}

template <int NB, int TC>
static void launch_chunk_kernel(dim3 grid, dim3 block, size_t lds, const AttnCArgs& a, hipStream_t s) {
    static size_t lds_set = 65536;   // dynamic LDS above 64 KB must be allowed first
    if (lds > lds_set) {
        L3P_HIP(hipFuncSetAttribute((const void*)attn_chunk_kernel<NB, TC>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)lds));
        lds_set = lds;
    }
    hipLaunchKernelGGL((attn_chunk_kernel<NB, TC>), grid, block, lds, s, a);
    L3P_HIP(hipGetLastError());
}

// Chunk and merge launches for `tokens` tokens of up to `chunks` chunks each.
static void launch_chunks(const Model& m, const AttnCArgs& a, int chunks, int tokens, hipStream_t s) {
    const int tc = a.tc;
    const int rowdw = chunk_rows_dw(tc, m.hq8);
    const size_t lds = (size_t)m.kv_mul * m.hs * 4 + 2 * (size_t)m.hs * 4 + (size_t)m.kv_mul * 8 * tc * 4 +
                       (size_t)m.kv_mul * m.hs + (size_t)m.kv_mul * 8 * 4 + 3 * (size_t)m.hs * 4 +
                       2 * (size_t)rowdw * 4 + 16;
    const dim3 grid(m.n_kv, chunks, tokens), block(64 * m.kv_mul);
    L3P_REQUIRE(tc == kTC || (tc == 32 && m.hs >= 192), L3P_E_INVALID, "attention: chunk of %d positions", tc);
    switch (m.hs / 32) {
    case 1: launch_chunk_kernel<1, kTC>(grid, block, lds, a, s); break;
    case 2: launch_chunk_kernel<2, kTC>(grid, block, lds, a, s); break;
    case 3: launch_chunk_kernel<3, kTC>(grid, block, lds, a, s); break;
    case 4: launch_chunk_kernel<4, kTC>(grid, block, lds, a, s); break;
    case 5: launch_chunk_kernel<5, kTC>(grid, block, lds, a, s); break;
    case 6:
        if (tc == 32) launch_chunk_kernel<6, 32>(grid, block, lds, a, s);
        else launch_chunk_kernel<6, kTC>(grid, block, lds, a, s);
        break;
    case 7:
        if (tc == 32) launch_chunk_kernel<7, 32>(grid, block, lds, a, s);
        else launch_chunk_kernel<7, kTC>(grid, block, lds, a, s);
        break;
    default:
        if (tc == 32) launch_chunk_kernel<8, 32>(grid, block, lds, a, s);
        else launch_chunk_kernel<8, kTC>(grid, block, lds, a, s);
        break;
    }
    const dim3 mgrid(m.n_heads, tokens);
    switch (m.hs / 32) {
    case 1: hipLaunchKernelGGL(attn_merge_kernel<1>, mgrid, dim3(64), 0, s, a); break;
    case 2: hipLaunchKernelGGL(attn_merge_kernel<2>, mgrid, dim3(64), 0, s, a); break;
    case 3: hipLaunchKernelGGL(attn_merge_kernel<3>, mgrid, dim3(64), 0, s, a); break;
    case 4: hipLaunchKernelGGL(attn_merge_kernel<4>, mgrid, dim3(64), 0, s, a); break;
    case 5: hipLaunchKernelGGL(attn_merge_kernel<5>, mgrid, dim3(64), 0, s, a); break;
    case 6: hipLaunchKernelGGL(attn_merge_kernel<6>, mgrid, dim3(64), 0, s, a); break;
    case 7: hipLaunchKernelGGL(attn_merge_kernel<7>, mgrid, dim3(64), 0, s, a); break;
    default: hipLaunchKernelGGL(attn_merge_kernel<8>, mgrid, dim3(64), 0, s, a); break;
    }
    L3P_HIP(hipGetLastError());
}

template <int NB>
static void launch_head(const Model& m, const AttnCArgs& a, hipStream_t s) {
    const size_t lds = (size_t)kHW * 2 * kHSlot + (size_t)kHW * (32 * NB + 2) * 4 + 256 + 32 + 2 * (size_t)((34 * NB + 3) & ~3);
    static size_t lds_set = 65536;   // dynamic LDS above 64 KB must be allowed first
    if (lds > lds_set) {
        L3P_HIP(hipFuncSetAttribute((const void*)attn_head_kernel<NB>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        lds_set = lds;
    }
    hipLaunchKernelGGL(attn_head_kernel<NB>, dim3(m.n_heads), dim3(64 * kHW), lds, s, a);
    L3P_HIP(hipGetLastError());
}

void launch_attention(const Model& m, int l, const AttnIO& io, bool per_head, hipStream_t s) {
    AttnCArgs a = attn_args(m, l, io);
    if (!per_head) {
        a.tc = m.dec_tc;   // part_chunks = max_chunks counts chunks of dec_tc positions
        launch_chunks(m, a, m.max_chunks, 1, s);
        return;
    }
    switch (m.hs / 32) {
    case 1: launch_head<1>(m, a, s); break;
    case 2: launch_head<2>(m, a, s); break;
    case 3: launch_head<3>(m, a, s); break;
    case 4: launch_head<4>(m, a, s); break;
    case 5: launch_head<5>(m, a, s); break;
    case 6: launch_head<6>(m, a, s); break;
    case 7: launch_head<7>(m, a, s); break;
    default: launch_head<8>(m, a, s); break;
    }
}

// Prompt batches take attn_prefill_kernel when its LDS fits a CU
// (L3P_PREFILL_ATTN=chunks keeps them on the chunk + merge kernels).
static bool prefill_attention_fits(const Model& m) {
    const char* e = getenv("L3P_PREFILL_ATTN");
    if (e && strcmp(e, "chunks") == 0) return false;
    return prefill_attn_lds(m.hs / 32, m.kv_mul) <= 160 * 1024;
}

template <int NB, int WPH>
static void launch_prefill_attn_w(const Model& m, const AttnCArgs& a, int tokens, size_t lds, hipStream_t s) {
    static size_t lds_set = 65536;   // dynamic LDS above 64 KB must be allowed first
    if (lds > lds_set) {
        L3P_HIP(hipFuncSetAttribute((const void*)attn_prefill_kernel<NB, WPH>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        lds_set = lds;
    }
    hipLaunchKernelGGL((attn_prefill_kernel<NB, WPH>), dim3(m.n_kv, (tokens + kPT - 1) / kPT),
                       dim3(64 * m.kv_mul * WPH), lds, s, a, tokens);
    L3P_HIP(hipGetLastError());
}

// Two waves per head when the group's threads stay within 1024 and the
// second parts' states fit the copy buffers for the final merge.
template <int NB>
static void launch_prefill_attn(const Model& m, const AttnCArgs& a, int tokens, hipStream_t s) {
    const size_t lds = prefill_attn_lds(NB, m.kv_mul);
    const size_t merge = (size_t)m.kv_mul * 64 * (2 + 8 * NB) * 4;
    const size_t raw = 4 * (size_t)prefill_raw_dwords(34 * NB) * 4;
    if (m.kv_mul <= 8 && merge <= raw) launch_prefill_attn_w<NB, 2>(m, a, tokens, lds, s);
    else launch_prefill_attn_w<NB, 1>(m, a, tokens, lds, s);
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
    a.rope = nullptr;   // each token's RoPE rows come from the tables at its position
    a.part = part;
    a.part_chunks = chunks;
    a.part_stride = (size_t)m.n_heads * chunks * attn_part_row(m.hs);
    L3P_REQUIRE(a.part_stride * tokens <= part_cap, L3P_E_INVALID, "attention: %d tokens exceed the partials buffer",
                tokens);
    hipLaunchKernelGGL(kv_rows_kernel, dim3(m.n_kv, tokens), dim3(64), 0, s, a);
    L3P_HIP(hipGetLastError());
    if (prefill_attention_fits(m)) {
        switch (m.hs / 32) {
        case 1: launch_prefill_attn<1>(m, a, tokens, s); break;
        case 2: launch_prefill_attn<2>(m, a, tokens, s); break;
        case 3: launch_prefill_attn<3>(m, a, tokens, s); break;
        case 4: launch_prefill_attn<4>(m, a, tokens, s); break;
        case 5: launch_prefill_attn<5>(m, a, tokens, s); break;
        case 6: launch_prefill_attn<6>(m, a, tokens, s); break;
        case 7: launch_prefill_attn<7>(m, a, tokens, s); break;
        default: launch_prefill_attn<8>(m, a, tokens, s); break;
        }
        return;
    }
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

template <int R>
static void launch_topk_scan(const float* l, int n, int k, const float* gmax, int ng, float* out_v, int* out_i,
                             hipStream_t s, HostSlots pub) {
    const size_t lds = (2 * (size_t)kScanBlock + 2 * 256) * 4;
    static bool lds_set = false;   // dynamic LDS above 64 KB must be allowed first
    if (!lds_set) {
        L3P_HIP(hipFuncSetAttribute((const void*)topk_scan_kernel<R>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)lds));
        lds_set = true;
    }
    hipLaunchKernelGGL(topk_scan_kernel<R>, dim3(1), dim3(1024), lds, s, l, n, k, gmax, ng, out_v, out_i, pub);
    L3P_HIP(hipGetLastError());
}

void launch_topk_slots(const float* l, int n, int k, float* gmax, float* out_v, int* out_i, hipStream_t s,
                       HostSlots pub) {
    L3P_REQUIRE(k >= 1 && k <= 64 * kSlotsPerLane && k <= n, L3P_E_UNSUPPORTED, "sampler: top_k=%d outside [1, %d]",
                k, 64 * kSlotsPerLane);
    const int ng = sample_groups(n);
    hipLaunchKernelGGL(topk_groupmax_kernel, dim3((ng + 15) / 16), dim3(1024), 0, s, l, n, k, ng, gmax);
    L3P_HIP(hipGetLastError());
    const int rows = (k + 63) / 64;
    if (rows <= 1) launch_topk_scan<1>(l, n, k, gmax, ng, out_v, out_i, s, pub);
    else if (rows <= 2) launch_topk_scan<2>(l, n, k, gmax, ng, out_v, out_i, s, pub);
    else if (rows <= 4) launch_topk_scan<4>(l, n, k, gmax, ng, out_v, out_i, s, pub);
    else launch_topk_scan<kSlotsPerLane>(l, n, k, gmax, ng, out_v, out_i, s, pub);
}
