// gemv.hip — decode GEMVs over GGUF blocks in their native layout (gfx950).
//
// One workgroup owns a tile of R consecutive rows of a matrix and the whole
// K extent.  Thread t owns block column t (32 consecutive inputs; for K-quants
// the 32-input sub-block t), keeps its 32 inputs of x in registers and walks
// the R rows of the tile:
//
//   1. the tile, R*row_bytes contiguous bytes of HBM, is copied into LDS with
//      coalesced 16-byte loads (rows are 16-byte multiples for every shape of
//      the Llama-3 / Gemma dimensions);
//   2. each thread reads its block of every row back from LDS as aligned
//      dwords and realigns it in registers (Q8_0 and Q4_0 blocks are 34 and
//      18 bytes, so odd columns start 2 bytes into a dword);
//   3. partial sums are reduced across the workgroup (wave butterfly, then a
//      fixed-order sum over waves), so results are deterministic.
//
// Arithmetic per type follows the reference's matmul_quantized dispatch
// (llama3pure-c-engine.c:2091-2133): Q8_0/Q4_K/Q6_K weights are dequantized
// exactly and multiplied with fp32 x (matmul_deq_4row, c:2136-2176); Q4_0
// takes x quantized to Q8_0 and exact integer block dots (c:1625-1643).
// Only the fp32 summation order differs from the reference's sequential loop.
#include "device_common.h"
#include "internal.h"

namespace {

constexpr int kMaxThreads = 1024;

using namespace l3pd;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Copy `nbytes` (a multiple of 4) from 16-byte aligned global memory to LDS.
// Weights are streamed once per call, so the loads are marked non-temporal.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void tile_to_lds(uint32_t* lds, const uint8_t* __restrict__ src, int nbytes,
                                            int t, int nt) {
    const int n16 = nbytes >> 4;
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
    u32x4* d = reinterpret_cast<u32x4*>(lds);
    int c = t;
    for (; c + 3 * nt < n16; c += 4 * nt) {
        u32x4 a0 = __builtin_nontemporal_load(s + c);
        u32x4 a1 = __builtin_nontemporal_load(s + c + nt);
        u32x4 a2 = __builtin_nontemporal_load(s + c + 2 * nt);
        u32x4 a3 = __builtin_nontemporal_load(s + c + 3 * nt);
        d[c] = a0;
        d[c + nt] = a1;
        d[c + 2 * nt] = a2;
        d[c + 3 * nt] = a3;
    }
    for (; c < n16; c += nt) d[c] = __builtin_nontemporal_load(s + c);
    const int rem = (nbytes & 15) >> 2;
    if (t < rem) lds[(n16 << 2) + t] = reinterpret_cast<const uint32_t*>(src)[(n16 << 2) + t];
}

// Locate the workgroup's segment and first row.  In pair mode both segments
// share the row range.
struct TileLoc {
    int seg, r0, nr;
};
template <int R, bool PAIR>
__device__ __forceinline__ TileLoc locate(const GemvBatch& B) {
    int bid = blockIdx.x, s = 0;
    if (!PAIR) {
        while (s < B.nseg - 1) {
            int nt = (B.seg[s].rows + R - 1) / R;
            if (bid < nt) break;
            bid -= nt;
            ++s;
        }
    }
    TileLoc L;
    L.seg = s;
    L.r0 = bid * R;
    L.nr = min(R, B.seg[s].rows - L.r0);
    return L;
}

// Reduce acc[NRR] over the workgroup and apply the epilogue.
template <int R, bool PAIR>
__device__ __forceinline__ void finish(const GemvBatch& B, const TileLoc& L, float* acc, float* red) {
    constexpr int NRR = PAIR ? 2 * R : R;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int i = 0; i < NRR; ++i) {
        float v = wave_sum(acc[i]);
        if (lane == 0) red[w * NRR + i] = v;
    }
    __syncthreads();
    if (t < L.nr) {
        float a = 0.0f, b = 0.0f;
        for (int k = 0; k < nw; ++k) {
            a += red[k * NRR + t];
            if (PAIR) b += red[k * NRR + R + t];
        }
        const int r = L.r0 + t;
        if (PAIR) {
            B.seg[0].y[r] = B.epilogue == EPI_GEGLU ? ref_geglu(a, b) : ref_swiglu(a, b);
        } else {
            float* y = B.seg[L.seg].y;
            if (B.epilogue == EPI_ADD) y[r] += a;
            else y[r] = a;
        }
    }
}

// ---------------------------------------------------------------------------
// Q8_0: 34-byte blocks {fp16 d; int8 q[32]} (c:127-130), w = q*d exactly.
// ---------------------------------------------------------------------------
template <int R, bool PAIR>
__global__ void __launch_bounds__(kMaxThreads) gemv_q8_0_kernel(GemvBatch B, int cols,
                                                                 const float* __restrict__ x) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int NRR = PAIR ? 2 * R : R;
    const int nb = cols >> 5;
    const uint32_t rb = (uint32_t)nb * 34u;
    const int t = threadIdx.x, nt = blockDim.x;
    const TileLoc L = locate<R, PAIR>(B);

    tile_to_lds(lds, B.seg[L.seg].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);
    if (PAIR) tile_to_lds(lds + (R * rb >> 2), B.seg[1].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);

    const bool active = t < nb;
    float xv[32];
    if (active) {
        const float4* xp = reinterpret_cast<const float4*>(x + 32 * t);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float4 v = xp[k];
            xv[4 * k] = v.x; xv[4 * k + 1] = v.y; xv[4 * k + 2] = v.z; xv[4 * k + 3] = v.w;
        }
    }
    __syncthreads();

    float acc[NRR];
    // Even columns start dword-aligned: d in the low half, quants 2 bytes in.
    // Odd columns start 2 bytes into a dword: d in the high half, quants
    // dword-aligned one dword later.
    const uint32_t qsh = (t & 1) ? 32u : 16u;
    const uint32_t dsh = (t & 1) ? 16u : 0u;
#pragma unroll
    for (int i = 0; i < NRR; ++i) {
        float a = 0.0f;
        if (active && (i % R) < L.nr) {
            const uint32_t E = ((uint32_t)i * rb + 34u * (uint32_t)t) >> 2;
            uint32_t dw[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) dw[k] = lds[E + k];
            const float d = h2f(dw[0] >> dsh);
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t q = shr64(dw[k], dw[k + 1], qsh);
                s0 = fmaf((float)(int8_t)(q), xv[4 * k + 0], s0);
                s1 = fmaf((float)(int8_t)(q >> 8), xv[4 * k + 1], s1);
                s0 = fmaf((float)(int8_t)(q >> 16), xv[4 * k + 2], s0);
                s1 = fmaf((float)(int8_t)(q >> 24), xv[4 * k + 3], s1);
            }
            a = (s0 + s1) * d;
        }
        acc[i] = a;
    }
    float* red = reinterpret_cast<float*>(lds) + ((PAIR ? 2 : 1) * R * rb + 15) / 16 * 4;
    finish<R, PAIR>(B, L, acc, red);
}

// ---------------------------------------------------------------------------
// Q4_0: 18-byte blocks {fp16 d; u8 qs[16]} (c:151-154) against Q8_0 x.
// Per block: isum = sum xq*(q-8) exactly, term = dw*dx*(float)isum
// (vec_dot_q4_0_q8_0, c:1625-1643).
// ---------------------------------------------------------------------------
template <int R, bool PAIR>
__global__ void __launch_bounds__(kMaxThreads) gemv_q4_0_kernel(GemvBatch B, int cols, XQ8 xq) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int NRR = PAIR ? 2 * R : R;
    const int nb = cols >> 5;
    const uint32_t rb = (uint32_t)nb * 18u;
    const int t = threadIdx.x, nt = blockDim.x;
    const TileLoc L = locate<R, PAIR>(B);

    tile_to_lds(lds, B.seg[L.seg].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);
    if (PAIR) tile_to_lds(lds + (R * rb >> 2), B.seg[1].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);

    const bool active = t < nb;
    int xw[8];
    float dx = 0.0f;
    int xsum8 = 0;
    if (active) {
        const int4* xp = reinterpret_cast<const int4*>(xq.qs + 32 * t);
        int4 a = xp[0], b = xp[1];
        xw[0] = a.x; xw[1] = a.y; xw[2] = a.z; xw[3] = a.w;
        xw[4] = b.x; xw[5] = b.y; xw[6] = b.z; xw[7] = b.w;
        dx = xq.d[t];
        xsum8 = 8 * xq.sum[t];
    }
    __syncthreads();

    float acc[NRR];
    const uint32_t qsh = (t & 1) ? 32u : 16u;
    const uint32_t dsh = (t & 1) ? 16u : 0u;
#pragma unroll
    for (int i = 0; i < NRR; ++i) {
        float a = 0.0f;
        if (active && (i % R) < L.nr) {
            const uint32_t E = ((uint32_t)i * rb + 18u * (uint32_t)t) >> 2;
            uint32_t dw[5];
#pragma unroll
            for (int k = 0; k < 5; ++k) dw[k] = lds[E + k];
            const float dw16 = h2f(dw[0] >> dsh);
            int isum = -xsum8;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = shr64(dw[k], dw[k + 1], qsh);
                isum = __builtin_amdgcn_sdot4((int)(q & 0x0f0f0f0fu), xw[k], isum, false);
                isum = __builtin_amdgcn_sdot4((int)((q >> 4) & 0x0f0f0f0fu), xw[4 + k], isum, false);
            }
            a = dw16 * dx * (float)isum;
        }
        acc[i] = a;
    }
    float* red = reinterpret_cast<float*>(lds) + ((PAIR ? 2 : 1) * R * rb + 15) / 16 * 4;
    finish<R, PAIR>(B, L, acc, red);
}

// ---------------------------------------------------------------------------
// Q4_K: 144-byte super-blocks {fp16 d, dmin; u8 scales[12]; u8 qs[128]}
// (c:157-162), 8 sub-blocks of 32 with 6-bit scale/min (c:705-746):
// w = (d*sc)*q - dmin*m.  Thread t owns sub-block j = t%8 of super-block
// t/8 and evaluates d1*sum(q*x) - m1*sum(x), with d1 = d*sc and m1 =
// dmin*m exact products.
// ---------------------------------------------------------------------------
template <int R, bool PAIR>
__global__ void __launch_bounds__(kMaxThreads) gemv_q4_k_kernel(GemvBatch B, int cols,
                                                                 const float* __restrict__ x) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int NRR = PAIR ? 2 * R : R;
    const int nsub = cols >> 5;
    const uint32_t rb = (uint32_t)(cols >> 8) * 144u;
    const int t = threadIdx.x, nt = blockDim.x;
    const TileLoc L = locate<R, PAIR>(B);

    tile_to_lds(lds, B.seg[L.seg].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);
    if (PAIR) tile_to_lds(lds + (R * rb >> 2), B.seg[1].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);

    const bool active = t < nsub;
    const int j = t & 7;           // sub-block within the super-block
    const int sb = t >> 3;
    float xv[32];
    float xs = 0.0f;
    if (active) {
        const float4* xp = reinterpret_cast<const float4*>(x + 32 * t);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float4 v = xp[k];
            xv[4 * k] = v.x; xv[4 * k + 1] = v.y; xv[4 * k + 2] = v.z; xv[4 * k + 3] = v.w;
        }
#pragma unroll
        for (int k = 0; k < 32; ++k) xs += xv[k];
    }
    __syncthreads();

    float acc[NRR];
    const uint32_t nsh = (j & 1) ? 4u : 0u;
#pragma unroll
    for (int i = 0; i < NRR; ++i) {
        float a = 0.0f;
        if (active && (i % R) < L.nr) {
            const uint32_t E = ((uint32_t)i * rb + 144u * (uint32_t)sb) >> 2;
            const uint4 hdr = *reinterpret_cast<const uint4*>(lds + E);   // d,dmin,scales[12]
            const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
            // 6-bit scale/min of sub-block j (get_scale_min_k4, c:705-714)
            const uint32_t bs = 8u * (uint32_t)(j & 3);
            const uint32_t b0 = (hdr.y >> bs) & 0xffu, b1 = (hdr.z >> bs) & 0xffu, b2 = (hdr.w >> bs) & 0xffu;
            const uint32_t sc = j < 4 ? (b0 & 63u) : ((b2 & 0x0fu) | ((b0 >> 6) << 4));
            const uint32_t mn = j < 4 ? (b1 & 63u) : ((b2 >> 4) | ((b1 >> 6) << 4));
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            const uint4* qp = reinterpret_cast<const uint4*>(lds + E + 4 + 8 * (j >> 1));
            const uint4 qa = qp[0], qb = qp[1];
            const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t q = (qw[k] >> nsh) & 0x0f0f0f0fu;
                s0 = fmaf((float)(q & 0xffu), xv[4 * k + 0], s0);
                s1 = fmaf((float)((q >> 8) & 0xffu), xv[4 * k + 1], s1);
                s0 = fmaf((float)((q >> 16) & 0xffu), xv[4 * k + 2], s0);
                s1 = fmaf((float)(q >> 24), xv[4 * k + 3], s1);
            }
            a = d1 * (s0 + s1) - m1 * xs;
        }
        acc[i] = a;
    }
    float* red = reinterpret_cast<float*>(lds) + ((PAIR ? 2 : 1) * R * rb + 15) / 16 * 4;
    finish<R, PAIR>(B, L, acc, red);
}

// ---------------------------------------------------------------------------
// Q6_K: 210-byte super-blocks {u8 ql[128]; u8 qh[64]; i8 sc[16]; fp16 d}
// (c:190-195), w = d*sc*(q-32) exactly (c:873-904).  Thread t owns, in
// super-block t/8, half h = (t%8)/4 and l in [8c, 8c+8) with c = t%4: four
// runs of 8 elements (offsets 0, 32, 64, 96 of the half), each run sharing
// one sub-scale.  Per run: (d*sc) * (sum(q*x) - 32*sum(x)).
// ---------------------------------------------------------------------------
template <int R, bool PAIR>
__global__ void __launch_bounds__(kMaxThreads) gemv_q6_k_kernel(GemvBatch B, int cols,
                                                                 const float* __restrict__ x) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int NRR = PAIR ? 2 * R : R;
    const int nthr = cols >> 5;
    const uint32_t rb = (uint32_t)(cols >> 8) * 210u;
    const int t = threadIdx.x, nt = blockDim.x;
    const TileLoc L = locate<R, PAIR>(B);

    tile_to_lds(lds, B.seg[L.seg].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);
    if (PAIR) tile_to_lds(lds + (R * rb >> 2), B.seg[1].w + (size_t)L.r0 * rb, L.nr * rb, t, nt);

    const bool active = t < nthr;
    const int sb = t >> 3, h = (t >> 2) & 1, c = t & 3;
    float xv[32];     // xv[8*g + e] = x[256*sb + 128*h + 32*g + 8*c + e]
    float xs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (active) {
        const float* xb = x + 256 * sb + 128 * h + 8 * c;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4* xp = reinterpret_cast<const float4*>(xb + 32 * g);
            float4 v0 = xp[0], v1 = xp[1];
            xv[8 * g + 0] = v0.x; xv[8 * g + 1] = v0.y; xv[8 * g + 2] = v0.z; xv[8 * g + 3] = v0.w;
            xv[8 * g + 4] = v1.x; xv[8 * g + 5] = v1.y; xv[8 * g + 6] = v1.z; xv[8 * g + 7] = v1.w;
#pragma unroll
            for (int e = 0; e < 8; ++e) xs[g] += xv[8 * g + e];
        }
    }
    __syncthreads();

    float acc[NRR];
#pragma unroll
    for (int i = 0; i < NRR; ++i) {
        float a = 0.0f;
        if (active && (i % R) < L.nr) {
            const uint32_t base = (uint32_t)i * rb + 210u * (uint32_t)sb;   // even bytes
            const uint32_t sh = (base & 2u) ? 16u : 0u;
            // 2-dword loads realigned: ql[64h+8c..+8], ql[64h+32+8c..+8], qh[32h+8c..+8]
            auto ld2 = [&](uint32_t byteoff, uint32_t& lo, uint32_t& hi) {
                const uint32_t E = (base + byteoff) >> 2;
                const uint32_t a0 = lds[E], a1 = lds[E + 1], a2 = lds[E + 2];
                lo = shr64(a0, a1, sh);
                hi = shr64(a1, a2, sh);
            };
            uint32_t la0, la1, lb0, lb1, h0, h1;
            ld2(64u * h + 8u * c, la0, la1);
            ld2(64u * h + 32u + 8u * c, lb0, lb1);
            ld2(128u + 32u * h + 8u * c, h0, h1);
            uint32_t s0w, s1w, dd;
            {
                // scales sc[8h + c/2 + {0,2,4,6}] and d at byte 208
                const uint32_t E = (base + 192u) >> 2;
                const uint32_t a0 = lds[E], a1 = lds[E + 1], a2 = lds[E + 2], a3 = lds[E + 3],
                               a4 = lds[E + 4];
                const uint32_t w0 = shr64(a0, a1, sh), w1 = shr64(a1, a2, sh), w2 = shr64(a2, a3, sh),
                               w3 = shr64(a3, a4, sh);
                // bytes 192..207 = sc[0..15] in w0..w3; bytes 208..209 = d in low half of next
                s0w = h ? w2 : w0;
                s1w = h ? w3 : w1;
                dd = a4 >> sh;
            }
            const float d = h2f(dd);
            const int cs = c >> 1;
            // sc index within the half: cs + 2g  -> byte (cs + 2g) of (s0w, s1w)
            auto scv = [&](int g) -> float {
                const int k = cs + 2 * g;
                const uint32_t w = k < 4 ? s0w : s1w;
                return (float)(int8_t)(w >> (8 * (k & 3)));
            };
            const uint32_t ql[4][2] = {{la0, la1}, {lb0, lb1}, {la0 >> 4, la1 >> 4}, {lb0 >> 4, lb1 >> 4}};
            float tot = 0.0f;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float s = 0.0f;
#pragma unroll
                for (int hw = 0; hw < 2; ++hw) {
                    const uint32_t hb = hw ? h1 : h0;
                    const uint32_t q = (ql[g][hw] & 0x0f0f0f0fu) | (((hb >> (2 * g)) & 0x03030303u) << 4);
                    s = fmaf((float)(q & 0xffu), xv[8 * g + 4 * hw + 0], s);
                    s = fmaf((float)((q >> 8) & 0xffu), xv[8 * g + 4 * hw + 1], s);
                    s = fmaf((float)((q >> 16) & 0xffu), xv[8 * g + 4 * hw + 2], s);
                    s = fmaf((float)(q >> 24), xv[8 * g + 4 * hw + 3], s);
                }
                tot = fmaf(d * scv(g), s - 32.0f * xs[g], tot);
            }
            a = tot;
        }
        acc[i] = a;
    }
    float* red = reinterpret_cast<float*>(lds) + ((PAIR ? 2 : 1) * R * rb + 15) / 16 * 4;
    finish<R, PAIR>(B, L, acc, red);
}

// ---------------------------------------------------------------------------
// Activation quantization (quantize_row_q8_0, c:1508-1528), bit-exact.
// ---------------------------------------------------------------------------
__global__ void quantize_x_kernel(const float* __restrict__ x, int nb, XQ8 out) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = x[32 * b + j];
    QBlock qb;
    quantize32(v, qb);
    int4* dst = reinterpret_cast<int4*>(out.qs + 32 * b);
    const int* qi = reinterpret_cast<const int*>(qb.q);
    dst[0] = make_int4(qi[0], qi[1], qi[2], qi[3]);
    dst[1] = make_int4(qi[4], qi[5], qi[6], qi[7]);
    out.d[b] = h2f_exact(qb.dh);
    out.sum[b] = qb.sum;
}

__global__ void quantize_blocks_kernel(const float* __restrict__ x, int64_t nb, uint8_t* __restrict__ dst) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = x[32 * b + j];
    QBlock qb;
    quantize32(v, qb);
    uint8_t* o = dst + 34 * b;
    o[0] = (uint8_t)(qb.dh & 0xff);
    o[1] = (uint8_t)(qb.dh >> 8);
#pragma unroll
    for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)qb.q[j];
}

// ---------------------------------------------------------------------------
// Dequantization, one element per thread, bit-exact with dequantize_row
// (c:611-934) for the types listed in l3p.h.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float ldh(const uint8_t* p) { return h2f_exact((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

__device__ float deq_elem(int type, const uint8_t* __restrict__ s, int64_t i) {
    switch (type) {
    case L3P_F32: return reinterpret_cast<const float*>(s)[i];
    case L3P_F16: return ldh(s + 2 * i);
    case L3P_BF16:
        return __uint_as_float(((uint32_t)s[2 * i] | ((uint32_t)s[2 * i + 1] << 8)) << 16);
    case L3P_Q4_0: {
        const uint8_t* b = s + (i >> 5) * 18;
        const int j = (int)(i & 31);
        const int q = j < 16 ? (b[2 + j] & 0x0f) : (b[2 + j - 16] >> 4);
        return (float)(q - 8) * ldh(b);
    }
    case L3P_Q4_1: {
        const uint8_t* b = s + (i >> 5) * 20;
        const int j = (int)(i & 31);
        const int q = j < 16 ? (b[4 + j] & 0x0f) : (b[4 + j - 16] >> 4);
        return (float)q * ldh(b) + ldh(b + 2);
    }
    case L3P_Q5_0: case L3P_Q5_1: {
        const bool one = type == L3P_Q5_1;
        const uint8_t* b = s + (i >> 5) * (one ? 24 : 22);
        const uint8_t* qhp = b + (one ? 4 : 2);
        const uint32_t qh = (uint32_t)qhp[0] | ((uint32_t)qhp[1] << 8) | ((uint32_t)qhp[2] << 16) |
                            ((uint32_t)qhp[3] << 24);
        const uint8_t* qs = qhp + 4;
        const int j = (int)(i & 31);
        const int q = j < 16 ? ((qs[j] & 0x0f) | (int)(((qh >> j) & 1u) << 4))
                             : ((qs[j - 16] >> 4) | (int)(((qh >> j) & 1u) << 4));
        return one ? (float)q * ldh(b) + ldh(b + 2) : (float)(q - 16) * ldh(b);
    }
    case L3P_Q8_0: {
        const uint8_t* b = s + (i >> 5) * 34;
        return (float)(int8_t)b[2 + (i & 31)] * ldh(b);
    }
    case L3P_IQ4_NL: {
        const int8_t kv[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
        const uint8_t* b = s + (i >> 5) * 18;
        const int j = (int)(i & 31);
        const int q = j < 16 ? (b[2 + j] & 0x0f) : (b[2 + j - 16] >> 4);
        return ldh(b) * (float)kv[q];
    }
    case L3P_Q4_K: {
        const uint8_t* b = s + (i >> 8) * 144;
        const int e = (int)(i & 255), g = e >> 6, hi = (e >> 5) & 1, l = e & 31;
        const int js = 2 * g + hi;
        const uint8_t* sc = b + 4;
        int scv, mnv;
        if (js < 4) {
            scv = sc[js] & 63;
            mnv = sc[js + 4] & 63;
        } else {
            scv = (sc[js + 4] & 0x0f) | ((sc[js - 4] >> 6) << 4);
            mnv = (sc[js + 4] >> 4) | ((sc[js] >> 6) << 4);
        }
        const float d1 = ldh(b) * (float)scv, m1 = ldh(b + 2) * (float)mnv;
        const int q = hi ? (b[16 + 32 * g + l] >> 4) : (b[16 + 32 * g + l] & 0x0f);
        return d1 * (float)q - m1;
    }
    case L3P_Q6_K: {
        const uint8_t* b = s + (i >> 8) * 210;
        const int e = (int)(i & 255), half = e >> 7, r = e & 127, g = r >> 5, l = r & 31;
        const uint8_t* ql = b + 64 * half;
        const uint8_t* qh = b + 128 + 32 * half;
        const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + 8 * half);
        const int lo = (g & 1) ? ql[l + 32] : ql[l];
        const int nib = (g & 2) ? (lo >> 4) : (lo & 0x0f);
        const int q = (nib | (((qh[l] >> (2 * g)) & 3) << 4)) - 32;
        return ldh(b + 208) * (float)sc[l / 16 + 2 * g] * (float)q;
    }
    default: return 0.0f;
    }
}

__global__ void dequant_kernel(int type, const uint8_t* __restrict__ s, int64_t n, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = deq_elem(type, s, i);
}

// Embedding row (c:3204-3207), times a scale when non-zero (Gemma's sqrt(dim),
// which the reference applies to x in place before the first norm,
// c:3132-3140; x*scale rounds the same), and the step record {token, pos}
// that the kernels of the step read.
__global__ void embed_step_kernel(int type, const uint8_t* __restrict__ s, int n, float scale, float* __restrict__ y,
                                  int token, int pos, int* step) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = deq_elem(type, s, i);
        y[i] = scale != 0.0f ? v * scale : v;
    }
    if (i == 0) {
        step[0] = token;
        step[1] = pos;
    }
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------
template <typename K>
void set_lds(K kern, size_t bytes) {
    if (bytes > 65536) L3P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
}

struct Shape {
    int threads;     // workgroup size
    uint32_t rb;     // row bytes
};

Shape shape_of(int type, int cols) {
    Shape s{0, (uint32_t)type_row_bytes(type, cols)};
    int lanes = 0;
    switch (type) {
    case L3P_Q8_0: case L3P_Q4_0: lanes = cols / 32; break;
    case L3P_Q4_K: case L3P_Q6_K: lanes = cols / 32; break;
    default: break;
    }
    s.threads = (lanes + 63) / 64 * 64;
    return s;
}

template <int R, bool PAIR>
void launch_typed(int type, const GemvBatch& b, int cols, const XPrep& xp, hipStream_t st) {
    const float* x = xp.x;
    const XQ8* xq = &xp.q8;
    const Shape sh = shape_of(type, cols);
    const int nrr = PAIR ? 2 * R : R;
    const size_t lds = ((size_t)(PAIR ? 2 : 1) * R * sh.rb + 15) / 16 * 16 + (size_t)(sh.threads / 64) * nrr * 4;
    int tiles = 0;
    if (PAIR) tiles = (b.seg[0].rows + R - 1) / R;
    else for (int s = 0; s < b.nseg; ++s) tiles += (b.seg[s].rows + R - 1) / R;
    if (tiles == 0) return;
    dim3 grid(tiles), block(sh.threads);
    switch (type) {
    case L3P_Q8_0:
        set_lds(gemv_q8_0_kernel<R, PAIR>, lds);
        hipLaunchKernelGGL((gemv_q8_0_kernel<R, PAIR>), grid, block, lds, st, b, cols, x);
        break;
    case L3P_Q4_0:
        set_lds(gemv_q4_0_kernel<R, PAIR>, lds);
        hipLaunchKernelGGL((gemv_q4_0_kernel<R, PAIR>), grid, block, lds, st, b, cols, *xq);
        break;
    case L3P_Q4_K:
        set_lds(gemv_q4_k_kernel<R, PAIR>, lds);
        hipLaunchKernelGGL((gemv_q4_k_kernel<R, PAIR>), grid, block, lds, st, b, cols, x);
        break;
    case L3P_Q6_K:
        set_lds(gemv_q6_k_kernel<R, PAIR>, lds);
        hipLaunchKernelGGL((gemv_q6_k_kernel<R, PAIR>), grid, block, lds, st, b, cols, x);
        break;
    default:
        throw L3pError{L3P_E_UNSUPPORTED, "gemv: unsupported type"};
    }
    L3P_HIP(hipGetLastError());
}

}  // namespace

bool gemv_supported(int type, int cols) {
    // Rows must be 16-byte multiples (tiles are copied with 16-byte loads and
    // every row then starts with the same dword alignment).
    switch (type) {
    case L3P_Q8_0: case L3P_Q4_0: case L3P_Q4_K: case L3P_Q6_K:
        return cols > 0 && cols % type_block_elems(type) == 0 && type_row_bytes(type, cols) % 16 == 0 &&
               cols / 32 <= kMaxThreads;
    default:
        return false;
    }
}

int gemv_input_form(int type, int cols) {
    (void)cols;
    return type == L3P_Q4_0 ? 1 : 0;
}

void launch_gemv(int type, const GemvBatch& b, int cols, const XPrep& xp, hipStream_t st) {
    L3P_REQUIRE(gemv_supported(type, cols), L3P_E_UNSUPPORTED, "gemv: type %d with %d columns not supported",
                type, cols);
    L3P_REQUIRE(type != L3P_Q4_0 || xp.q8.qs, L3P_E_INVALID, "gemv: Q4_0 needs the quantized activation");
    const size_t rb = type_row_bytes(type, cols);
    const bool pair = b.pair != 0;
    // Rows per tile: keep the LDS tile within 64 KB.
    const size_t tile_rows_budget = 65536 / ((pair ? 2 : 1) * rb);
    if (tile_rows_budget >= 4) {
        pair ? launch_typed<4, true>(type, b, cols, xp, st) : launch_typed<4, false>(type, b, cols, xp, st);
    } else if (tile_rows_budget >= 2) {
        pair ? launch_typed<2, true>(type, b, cols, xp, st) : launch_typed<2, false>(type, b, cols, xp, st);
    } else {
        pair ? launch_typed<1, true>(type, b, cols, xp, st) : launch_typed<1, false>(type, b, cols, xp, st);
    }
}

void prepare_x_form(int type, int cols, const float* x, const XPrep& xp, hipStream_t st) {
    switch (gemv_input_form(type, cols)) {
    case 1: launch_quantize_x(x, cols, xp.q8, st); break;
    default: break;
    }
}

void launch_quantize_x(const float* x, int cols, const XQ8& xq, hipStream_t st) {
    const int nb = cols / 32;
    hipLaunchKernelGGL(quantize_x_kernel, dim3((nb + 255) / 256), dim3(256), 0, st, x, nb, xq);
    L3P_HIP(hipGetLastError());
}

void launch_quantize_q8_0_blocks(const float* x, int64_t n, uint8_t* dst, hipStream_t st) {
    const int64_t nb = n / 32;
    if (nb == 0) return;
    hipLaunchKernelGGL(quantize_blocks_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, x, nb, dst);
    L3P_HIP(hipGetLastError());
}

void launch_dequant(int type, const uint8_t* src, int64_t n, float* dst, hipStream_t st) {
    if (n == 0) return;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, type, src, n, dst);
    L3P_HIP(hipGetLastError());
}

void launch_embed_row(int type, const uint8_t* row, int n, float scale, float* dst, int token, int pos, int* step,
                      hipStream_t st) {
    hipLaunchKernelGGL(embed_step_kernel, dim3((n + 255) / 256), dim3(256), 0, st, type, row, n, scale, dst, token,
                       pos, step);
    L3P_HIP(hipGetLastError());
}
