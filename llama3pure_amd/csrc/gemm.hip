// gemm.hip — the prefill GEMMs on the matrix cores (gfx950):
//   Y[m][n] (=|+=) sum_k W[n][k] * X[m][k]
// for M prompt tokens, N output features and K inputs, with W in its GGUF
// block layout.  They replace matmul_quantized_batch (llama3pure-c-engine.c:
// 2291-2331).  For the types the reference dequantizes before its batched dot
// (matmul_deq_batch_4row, c:2179-2273) the fp32 matrix cores multiply every
// weight expanded exactly to fp32 (dequantize_row_*, c:611-934) with the fp32
// activation, so the products are the reference's and only the fp32
// summation order differs.  For the types whose batched dot takes Q8_0
// activations (Q4_0, Q4_1, Q5_0, Q5_1, IQ4_NL) the int8 matrix cores form
// the exact block dots (the int8 section further down).
//
// Tiling.  A workgroup owns a 64 x BN tile of Y (BN = 64, or 128 for passes
// of at least 16 row tiles whose 128-wide tiles give every CU two workgroups
// without splitting K, so each X tile serves twice the outputs) and walks K
// in steps of 64:
//   1. the 64 x 64 X tile (fp32, from L2) and the dequantized BN x 64 W tile
//      go to LDS, rows padded to 68 floats; their global loads were issued
//      one step earlier, before that step's matrix work;
//   2. BN / 16 waves each compute a 32 x 32 block with v_mfma_f32_16x16x4_f32
//      (2 x 2 tiles of 16 x 16).  The instruction contracts over 4 k-slots,
//      slot g held by lanes 16g..16g+15; here slot g of step s is
//      k = kk + 4g + s, the same for A (X) and B (W), so each lane fetches
//      its four k values of a 16-wide slab with one ds_read_b128.
// Several workgroups per CU (a 1024-row prompt pass gives four per CU at
// N = 4096) and the one-step-ahead loads hide the load latency.
//
// One launch covers up to three matrices with the same K and X (q|k|v,
// gate|up): blockIdx.x runs over the N tiles of the segments in order.  When
// the tiles cannot give every CU four workgroups, the launch is stream-K:
// the (tile, K step) pairs, tile by tile, are cut into P equal runs for P
// resident workgroups, so every CU gets the same number of K steps (whole
// splits of K did not divide evenly: Gemma-2-2B's output and down
// projections gave 1152 workgroups of 8 and 36 steps for 1024 resident
// slots).  Each run writes its fp32 partial of each tile it touches to
// workspace slot j, j = its rank among the runs that share the tile, and
// gemm_reduce_kernel adds the slots in order, so results do not depend on
// scheduling.  (Splitting K over blockIdx.z, the same partials with equal
// splits, remains for workspaces too small for the stream-K slots.)
#include <algorithm>
#include <cstdlib>
#include <mutex>

#include "dequant.h"
#include "device_common.h"
#include "internal.h"

namespace {

using namespace l3pd;

constexpr int kBM = 64, kBK = 64;
constexpr int kLDK = kBK + 4;   // LDS row stride in floats (b128 reads spread over the banks)

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int int32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const uint8_t* w[3];   // per segment: weight rows,
    float* y[3];           // output rows [m][ldy],
    int ldy[3];
    int n[3];              // output features,
    int noff[3];           // first column in the split workspace's rows
    int tbeg[4];           // first N tile (tbeg[nseg] = all tiles)
    int nseg;
    size_t rb;             // bytes per weight row (same K and type for every segment)
    int k, m;              // inputs, batch rows
    const float* x;
    int ldx;
    int add;               // 1: Y += W.X (residual), 0: Y = W.X
    int nsplit, ksteps;    // K splits and kBK-steps per split
    float* part;           // [nsplit][m][ntot] partials when nsplit > 1
    int ntot;
    int streamk;           // > 0: stream-K over that many workgroups (grid.x), nsplit = most slots of a tile
    int kst;               // stream-K: kBK steps of a whole tile
    int bn;                // output columns per tile
};

// Stream-K bookkeeping: the runs of P workgroups cut the tile-major sequence
// of W (tile, K step) pairs at floor(p W / P); the run holding pair x is
// ((x + 1) P - 1) / W.
__host__ __device__ __forceinline__ int sk_owner(long x, long W, int P) {
    return (int)(((x + 1) * (long)P - 1) / W);
}

// One thread's slice of a step's W tile: row t / 4 of the tile, elements
// e0 .. e0 + 15 of that row with e0 = k0 + 16 (t % 4).  Sixteen consecutive
// elements lie in one Q8_0 block or one scale group of a K-quant, so the
// slice needs at most three 16-byte pieces and a few header words, which are
// fetched one step ahead like the X tile.
struct WRaw {
    uint4 a, b, c, d;       // quant bytes / header / F32 values, by type
    uint32_t h0, h1, h2;    // scale words and scale bytes, by type
};

__device__ __forceinline__ uint32_t byte_of(const uint4& u, int i) {   // byte i (0..15, not constant)
    const uint32_t w = i < 4 ? u.x : (i < 8 ? u.y : (i < 12 ? u.z : u.w));
    return (w >> (8 * (i & 3))) & 0xffu;
}
__device__ __forceinline__ uint32_t byte_c(const uint4& u, int j) {     // byte j (constant after unrolling)
    const uint32_t w = (j >> 2) == 0 ? u.x : ((j >> 2) == 1 ? u.y : ((j >> 2) == 2 ? u.z : u.w));
    return (w >> (8 * (j & 3))) & 0xffu;
}

template <int QT>
__device__ __forceinline__ void fetch_slice(WRaw& r, const uint8_t* row, int e0) {
    if constexpr (QT == L3P_Q8_0) {   // 34-byte blocks: d, 32 quants
        const uint8_t* b = row + (size_t)(e0 >> 5) * 34;
        r.h0 = *reinterpret_cast<const uint16_t*>(b);
        // 2-byte aligned: one unaligned 16-byte load, left untouched until
        // store_step so that nothing waits for it here
        __builtin_memcpy(&r.a, b + 2 + 16 * ((e0 >> 4) & 1), 16);
    } else if constexpr (QT == L3P_Q4_K) {   // 144 bytes: d, dmin, 12 scale bytes, 128 nibble pairs
        const uint8_t* b = row + (size_t)(e0 >> 8) * 144;
        const int e = e0 & 255;
        __builtin_memcpy(&r.b, b, 16);
        __builtin_memcpy(&r.a, b + 16 + 32 * (e >> 6) + (e & 31), 16);
    } else if constexpr (QT == L3P_Q5_K) {   // 176 bytes: d, dmin, 12 scale bytes, 32 high-bit bytes, 128 nibble pairs
        const uint8_t* b = row + (size_t)(e0 >> 8) * 176;
        const int e = e0 & 255;
        __builtin_memcpy(&r.c, b, 16);
        __builtin_memcpy(&r.b, b + 16 + (e & 31), 16);
        __builtin_memcpy(&r.a, b + 48 + 32 * (e >> 6) + (e & 31), 16);
    } else if constexpr (QT == L3P_Q6_K) {   // 210 bytes: ql[128], qh[64], 16 int8 scales, d
        const uint8_t* b = row + (size_t)(e0 >> 8) * 210;
        const int e = e0 & 255, half = e >> 7, g = (e & 127) >> 5, l0 = e & 31;
        __builtin_memcpy(&r.a, b + 64 * half + 32 * (g & 1) + l0, 16);
        __builtin_memcpy(&r.b, b + 128 + 32 * half + l0, 16);
        r.h0 = *reinterpret_cast<const uint16_t*>(b + 208);
        r.h1 = b[192 + 8 * half + (l0 >> 4) + 2 * g];
    } else if constexpr (QT == L3P_Q3_K) {   // 110 bytes: hmask[32], qs[64], 12 scale bytes, d
        const uint8_t* b = row + (size_t)(e0 >> 8) * 110;
        const int g = (e0 & 255) >> 4, half = g >> 3, second = g & 1;
        __builtin_memcpy(&r.a, b + 32 + 32 * half + 16 * second, 16);
        __builtin_memcpy(&r.b, b + 16 * second, 16);
        r.h0 = *reinterpret_cast<const uint16_t*>(b + 108);
        r.h1 = b[96 + (g & 7)];
        r.h2 = b[104 + (g & 3)];
    } else if constexpr (QT == L3P_Q2_K) {   // 84 bytes: 16 scale bytes, qs[64], d, dmin
        const uint8_t* b = row + (size_t)(e0 >> 8) * 84;
        const int g = (e0 & 255) >> 4, half = g >> 3, second = g & 1;
        __builtin_memcpy(&r.a, b + 16 + 32 * half + 16 * second, 16);
        __builtin_memcpy(&r.h0, b + 80, 4);
        r.h1 = b[g];
    } else if constexpr (QT == L3P_F16 || QT == L3P_BF16) {
        const uint4* p = reinterpret_cast<const uint4*>(row + 2 * (size_t)e0);
        r.a = p[0];
        r.b = p[1];
    } else {   // F32
        const uint4* p = reinterpret_cast<const uint4*>(row + 4 * (size_t)e0);
        r.a = p[0];
        r.b = p[1];
        r.c = p[2];
        r.d = p[3];
    }
}

// The slice's 16 values, each formed exactly as dequantize_row_* forms it
// (c:611-934; the expressions of deq_elem), from the fetched bytes.
template <int QT>
__device__ __forceinline__ void decode_slice(const WRaw& r, int e0, float (&v)[16]) {
    if constexpr (QT == L3P_Q8_0) {
        const float d = h2f_exact(r.h0);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = (float)(int8_t)byte_c(r.a, j) * d;
    } else if constexpr (QT == L3P_Q4_K || QT == L3P_Q5_K) {
        // sub-block js = e / 32 of the super-block: its 6-bit scale and min
        const uint4& hd = QT == L3P_Q4_K ? r.b : r.c;
        const int e = e0 & 255, js = e >> 5;
        int scv, mnv;
        if (js < 4) {
            scv = (int)(byte_of(hd, 4 + js) & 63u);
            mnv = (int)(byte_of(hd, 8 + js) & 63u);
        } else {
            scv = (int)((byte_of(hd, 8 + js) & 0x0fu) | ((byte_of(hd, js) >> 6) << 4));
            mnv = (int)((byte_of(hd, 8 + js) >> 4) | ((byte_of(hd, 4 + js) >> 6) << 4));
        }
        const float d1 = h2f_exact(hd.x & 0xffffu) * (float)scv, m1 = h2f_exact(hd.x >> 16) * (float)mnv;
        const int sh = QT == L3P_Q4_K ? 4 * ((e >> 5) & 1) : 4 * (js & 1);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int q = (int)((byte_c(r.a, j) >> sh) & 0x0fu);
            if constexpr (QT == L3P_Q5_K) q += ((byte_c(r.b, j) >> js) & 1u) ? 16 : 0;
            v[j] = d1 * (float)q - m1;
        }
    } else if constexpr (QT == L3P_Q6_K) {
        const int g = (e0 & 127) >> 5;
        const float ds = h2f_exact(r.h0) * (float)(int8_t)r.h1;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int lo = (int)byte_c(r.a, j);
            const int nib = (g & 2) ? (lo >> 4) : (lo & 0x0f);
            const int q = (nib | (int)(((byte_c(r.b, j) >> (2 * g)) & 3u) << 4)) - 32;
            v[j] = ds * (float)q;
        }
    } else if constexpr (QT == L3P_Q3_K) {
        const int g = (e0 & 255) >> 4, half = g >> 3, j4 = (g >> 1) & 3;
        const int lo = g < 8 ? (int)(r.h1 & 0x0fu) : (int)(r.h1 >> 4);
        const int sg = (lo | (int)(((r.h2 >> (2 * (g >> 2))) & 3u) << 4)) - 32;
        const float ds = h2f_exact(r.h0) * (float)sg;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int u = (int)((byte_c(r.a, j) >> (2 * j4)) & 3u);
            const int h = (int)((byte_c(r.b, j) >> (4 * half + j4)) & 1u);
            v[j] = ds * (float)(u - (h ? 0 : 4));
        }
    } else if constexpr (QT == L3P_Q2_K) {
        const int j4 = (((e0 & 255) >> 4) >> 1) & 3;
        const float dl = h2f_exact(r.h0 & 0xffffu) * (float)(r.h1 & 0x0fu);
        const float ml = h2f_exact(r.h0 >> 16) * (float)(r.h1 >> 4);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = dl * (float)((byte_c(r.a, j) >> (2 * j4)) & 3u) - ml;
    } else if constexpr (QT == L3P_F16 || QT == L3P_BF16) {
        const uint32_t hw[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t h = (hw[j >> 1] >> (16 * (j & 1))) & 0xffffu;
            v[j] = QT == L3P_F16 ? h2f_exact(h) : __uint_as_float(h << 16);
        }
    } else {   // F32
        const uint32_t fw[16] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w,
                                 r.c.x, r.c.y, r.c.z, r.c.w, r.d.x, r.d.y, r.d.z, r.d.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = __uint_as_float(fw[j]);
    }
}

// The global data of one K step, held in registers from the step before so
// that its loads are in flight while the matrix cores work on the current
// step: the X tile (4 float4 per thread) and this thread's W slice.
struct StepRegs {
    float4 x[4];   // the first 1024 / threads of them are used
    WRaw w;
};

template <int QT, int BN>
__device__ __forceinline__ void fetch_step(StepRegs& sr, const GemmArgs& a, const uint8_t* W, int N, int m0, int n0,
                                           int k0, int t) {
    constexpr int NT = 4 * BN, XU = 1024 / NT;   // threads; float4 of the X tile per thread
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const int i = t + NT * u, r = i >> 4, c = i & 15;
        const int m = m0 + r, kk = k0 + 4 * c;
        sr.x[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (m < a.m && kk < a.k) sr.x[u] = *reinterpret_cast<const float4*>(a.x + (size_t)m * a.ldx + kk);
    }
    const int n = n0 + (t >> 2), e0 = k0 + 16 * (t & 3);
    sr.w = WRaw{};
    if (n < N && e0 < a.k) fetch_slice<QT>(sr.w, W + (size_t)n * a.rb, e0);
}

// The step's tiles into LDS, rows padded to kLDK floats: X as fetched, W rows
// [n0, n0 + BN) x columns [k0, k0 + 64) dequantized exactly (slices past the
// matrix are zero bytes, whose values only meet zero X columns or rows that
// are not stored).
template <int QT, int BN>
__device__ __forceinline__ void store_step(float* xs, float* ws, const StepRegs& sr, int k0, int t) {
    constexpr int NT = 4 * BN, XU = 1024 / NT;
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const int i = t + NT * u, r = i >> 4, c = i & 15;
        *reinterpret_cast<float4*>(xs + r * kLDK + 4 * c) = sr.x[u];
    }
    float v[16];
    decode_slice<QT>(sr.w, k0 + 16 * (t & 3), v);
    float4* dst = reinterpret_cast<float4*>(ws + (t >> 2) * kLDK + 16 * (t & 3));
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
}

// The output tile a workgroup works on: segment, its weights and output
// features, first output feature and first batch row.
struct TileRef {
    int sg, N, n0, m0;
    const uint8_t* W;
};
template <int BN>
__device__ __forceinline__ TileRef tile_ref(const GemmArgs& a, int tile, int mtile) {
    TileRef r;
    r.sg = (a.nseg > 1 && tile >= a.tbeg[1]) ? ((a.nseg > 2 && tile >= a.tbeg[2]) ? 2 : 1) : 0;
    r.W = a.w[r.sg];
    r.N = a.n[r.sg];
    r.n0 = (tile - a.tbeg[r.sg]) * BN;
    r.m0 = mtile * kBM;
    return r;
}

// acc := this wave's 32 x 32 block of the tile's sum over K [kbeg, kend)
template <int QT, int BN>
__device__ __forceinline__ void tile_mma(const GemmArgs& a, const TileRef& tr, int kbeg, int kend, float* xs,
                                         float* ws, floatx4 (&acc)[2][2]) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    constexpr int WN = BN / 32;              // waves across N
    const int wm = w / WN, wn = w % WN;      // this wave's 32 x 32 block of the 64 x BN tile
    const int g = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int im = 0; im < 2; ++im)
#pragma unroll
        for (int in = 0; in < 2; ++in) acc[im][in] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    StepRegs sr;
    fetch_step<QT, BN>(sr, a, tr.W, tr.N, tr.m0, tr.n0, kbeg, t);
    for (int k0 = kbeg; k0 < kend; k0 += kBK) {
        store_step<QT, BN>(xs, ws, sr, k0, t);
        __syncthreads();
        // the next step's loads go out before this step's matrix work
        if (k0 + kBK < kend) fetch_step<QT, BN>(sr, a, tr.W, tr.N, tr.m0, tr.n0, k0 + kBK, t);
        // 128-wide tiles raise the wave's issue priority for its matrix work,
        // so that waves in their load and dequantization phase fill the gaps
        // (Llama-3-8B wo 4096 x 4096 at 1024 rows: 300 -> 274 us; at 64-wide
        // tiles it was slower); LLVM's MFMA / LDS-read interleaving strategy
        // 1 for 128-wide tiles and 0 for 64-wide ones (Gemma-2-2B down at 511
        // rows: 204 -> 197 us).  Neither changes an operation or its order.
        if (BN == 128) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            if constexpr (BN == 128) __builtin_amdgcn_iglp_opt(1);
            else __builtin_amdgcn_iglp_opt(0);
            float4 af[2], bf[2];
#pragma unroll
            for (int im = 0; im < 2; ++im)
                af[im] = *reinterpret_cast<const float4*>(xs + (32 * wm + 16 * im + i16) * kLDK + kk + 4 * g);
#pragma unroll
            for (int in = 0; in < 2; ++in)
                bf[in] = *reinterpret_cast<const float4*>(ws + (32 * wn + 16 * in + i16) * kLDK + kk + 4 * g);
            const float a0[4] = {af[0].x, af[0].y, af[0].z, af[0].w};
            const float a1[4] = {af[1].x, af[1].y, af[1].z, af[1].w};
            const float b0[4] = {bf[0].x, bf[0].y, bf[0].z, bf[0].w};
            const float b1[4] = {bf[1].x, bf[1].y, bf[1].z, bf[1].w};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[s], b0[s], acc[0][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[s], b1[s], acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[s], b0[s], acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[s], b1[s], acc[1][1], 0, 0, 0);
            }
        }
        if (BN == 128) __builtin_amdgcn_s_setprio(0);
        __syncthreads();
    }
}

// The tile's results: to Y (slot < 0) or to partial slot `slot`.
template <int BN>
__device__ __forceinline__ void tile_store(const GemmArgs& a, const TileRef& tr, int slot, const floatx4 (&acc)[2][2]) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    constexpr int WN = BN / 32;
    const int wm = w / WN, wn = w % WN;
    const int g = lane >> 4, i16 = lane & 15;
    // D layout of the 16 x 16 tile: lane (g, i16) holds rows 4g..4g+3 of column i16
    float* const Y = a.y[tr.sg];
    const int ldy = a.ldy[tr.sg];
    float* const P = slot >= 0 ? a.part + (size_t)slot * a.m * a.ntot + a.noff[tr.sg] : nullptr;
#pragma unroll
    for (int im = 0; im < 2; ++im)
#pragma unroll
        for (int in = 0; in < 2; ++in) {
            const int n = tr.n0 + 32 * wn + 16 * in + i16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = tr.m0 + 32 * wm + 16 * im + 4 * g + r;
                if (m < a.m && n < tr.N) {
                    const float v = acc[im][in][r];
                    if (slot >= 0) {
                        P[(size_t)m * a.ntot + n] = v;
                    } else {
                        float* p = Y + (size_t)m * ldy + n;
                        *p = a.add ? *p + v : v;
                    }
                }
            }
        }
}

template <int QT, int BN>
__global__ void __launch_bounds__(4 * BN) gemm_kernel(GemmArgs a) {
    __shared__ __align__(16) float xs[kBM * kLDK];
    __shared__ __align__(16) float ws[BN * kLDK];
    floatx4 acc[2][2];
    if (a.streamk) {
        // this workgroup's run [s0, s1) of the tile-major (tile, K step) pairs
        const int NT = a.tbeg[a.nseg], S = a.kst, P = (int)gridDim.x;
        const long W = (long)NT * ((a.m + kBM - 1) / kBM) * S;
        const long s1 = ((long)blockIdx.x + 1) * W / P;
        for (long s = (long)blockIdx.x * W / P; s < s1;) {
            const int tt = (int)(s / S), kb = (int)(s % S);
            const int ke = (int)min((long)S, kb + (s1 - s));
            const TileRef tr = tile_ref<BN>(a, tt % NT, tt / NT);
            tile_mma<QT, BN>(a, tr, kb * kBK, min(a.k, ke * kBK), xs, ws, acc);
            tile_store<BN>(a, tr, (int)blockIdx.x - sk_owner((long)tt * S, W, P), acc);
            s += ke - kb;
        }
        return;
    }
    const TileRef tr = tile_ref<BN>(a, blockIdx.x, blockIdx.y);
    const int kbeg = blockIdx.z * a.ksteps * kBK, kend = min(a.k, kbeg + a.ksteps * kBK);
    tile_mma<QT, BN>(a, tr, kbeg, kend, xs, ws, acc);
    tile_store<BN>(a, tr, a.nsplit > 1 ? (int)blockIdx.z : -1, acc);
}

// Y (=|+=) the sum of the K splits' partials, in split order (stream-K: the
// slots of the output's tile, in slot order): V consecutive outputs per
// thread (V = 4: 16-byte loads and stores where every segment's width, row
// stride and base allow them; each output's additions are the same either
// way), blockIdx.y = batch row.
template <int V>
__global__ void __launch_bounds__(256) gemm_reduce_kernel(GemmArgs a) {
    const int c = (blockIdx.x * 256 + threadIdx.x) * V, m = blockIdx.y;
    if (c >= a.ntot) return;
    const int sg = (a.nseg > 1 && c >= a.noff[1]) ? ((a.nseg > 2 && c >= a.noff[2]) ? 2 : 1) : 0;
    int nslot = a.nsplit;
    if (a.streamk) {   // the V outputs lie in one tile (V divides the tile width and the segment offsets)
        const int NT = a.tbeg[a.nseg], S = a.kst;
        const long W = (long)NT * ((a.m + kBM - 1) / kBM) * S;
        const long tt = (long)(m / kBM) * NT + a.tbeg[sg] + (c - a.noff[sg]) / a.bn;
        nslot = sk_owner((tt + 1) * S - 1, W, a.streamk) - sk_owner(tt * S, W, a.streamk) + 1;
    }
    const size_t zs = (size_t)a.m * a.ntot;
    float* y = a.y[sg] + (size_t)m * a.ldy[sg] + (c - a.noff[sg]);
    if constexpr (V == 4) {
        const float4* p = reinterpret_cast<const float4*>(a.part + (size_t)m * a.ntot + c);
        float4 v = p[0];
        for (int z = 1; z < nslot; ++z) {
            const float4 q = p[z * (zs / 4)];
            v.x += q.x;
            v.y += q.y;
            v.z += q.z;
            v.w += q.w;
        }
        float4* y4 = reinterpret_cast<float4*>(y);
        if (a.add) {
            const float4 o = *y4;
            v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
        }
        *y4 = v;
    } else {
        const float* p = a.part + (size_t)m * a.ntot + c;
        float v = p[0];
        for (int z = 1; z < nslot; ++z) v += p[z * zs];
        *y = a.add ? *y + v : v;
    }
}

template <int QT>
void launch_typed(const GemmArgs& a, int bn, hipStream_t st) {
    const dim3 grid = a.streamk ? dim3(a.streamk) : dim3(a.tbeg[a.nseg], (a.m + kBM - 1) / kBM, a.nsplit);
    if (bn == 128) launch_kernel(gemm_kernel<QT, 128>, grid, dim3(512), 0u, st, a);
    else launch_kernel(gemm_kernel<QT, 64>, grid, dim3(256), 0u, st, a);
}

}  // namespace

// The types the reference dequantizes before its batched dot
// (matmul_deq_batch_4row, c:2179-2273); Q4_0, Q4_1, Q5_0, Q5_1 and IQ4_NL
// take the Q8_0 activation path instead (exact integer block dots per row).
bool gemm_mfma_supported(int type) {
    switch (type) {
    case L3P_Q8_0: case L3P_Q2_K: case L3P_Q3_K: case L3P_Q4_K: case L3P_Q5_K: case L3P_Q6_K:
    case L3P_F16: case L3P_BF16: case L3P_F32: return true;
    default: return false;
    }
}

static int gemm_env(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? std::max(1, atoi(e)) : dflt;
}

// The launch plan of a job: K splits and the partials they need (floats).
GemmPlan gemm_plan(const GemmJob& j, size_t ws_floats) {
    GemmPlan p;
    int tiles = 0, tiles128 = 0, ntot = 0;
    for (int i = 0; i < j.nseg; ++i) {
        tiles += (j.seg[i].n + 63) / 64;
        tiles128 += (j.seg[i].n + 127) / 128;
        ntot += j.seg[i].n;
    }
    const int steps = (j.k + kBK - 1) / kBK;
    const int mt = (j.m + kBM - 1) / kBM;
    // 64 x 128 tiles (eight waves, half the X reads per output) for passes of
    // at least 16 row tiles whose 128-wide tiles give every CU two workgroups
    // unsplit (Llama-3-8B's 1024-row projections: MFMA busy 75 -> 77%, prompt
    // 130 -> 127 ms); otherwise 64 x 64 tiles (measured slower with 128 at
    // Gemma-2-2B's 511 rows: 25.2 -> 25.7 ms)
    if (mt >= 16 && (long)tiles128 * mt >= 2L * device_cus()) {
        p.bn = 128;
        p.ksteps = steps;
        p.nsplit = 1;
        return p;
    }
    // Stream-K while the tiles give fewer than four workgroups per CU (the
    // LDS of four fits a CU): as many workgroups as fit at once, each run at
    // least eight K steps long, when the workspace holds the slots
    // (L3P_GEMM_SK_BN = 128, L3P_GEMM_SK_WPC and L3P_GEMM_SK_MIN override the
    // tile width, the workgroups per CU and the shortest run, for measurement:
    // at Gemma-2-2B's 511 rows none of them was faster than these defaults)
    const int want = 4 * device_cus();
    if (ws_floats && j.m > 0 && (long)tiles * mt < want) {
        const int skbn = gemm_env("L3P_GEMM_SK_BN", 64) == 128 ? 128 : 64;
        const int skt = skbn == 128 ? tiles128 : tiles;
        const long W = (long)skt * mt * steps;
        const int P = (int)std::min<long>((long)gemm_env("L3P_GEMM_SK_WPC", skbn == 128 ? 3 : 4) * device_cus(),
                                          W / gemm_env("L3P_GEMM_SK_MIN", 8));
        if (P > skt * mt / 2 && P > 1) {   // fewer runs than tiles: plain tiles do as well
            int slots = 1;
            for (long tt = 0; tt < (long)skt * mt; ++tt)
                slots = std::max(slots, sk_owner((tt + 1) * steps - 1, W, P) - sk_owner(tt * steps, W, P) + 1);
            if ((size_t)slots * j.m * ntot <= ws_floats) {
                p.bn = skbn;
                p.streamk = P;
                p.ksteps = steps;
                p.nsplit = slots;
                p.partial_floats = (size_t)slots * j.m * ntot;
                return p;
            }
        }
    }
    // otherwise K splits, each at least eight K steps long
    int split = 1;
    if (ws_floats && j.m > 0 && (long)tiles * mt < want) {
        split = std::min({(int)((want + (long)tiles * mt - 1) / ((long)tiles * mt)), steps / 8, 8});
        while (split > 1 && (size_t)split * j.m * ntot > ws_floats) --split;
        split = std::max(split, 1);
    }
    p.ksteps = (steps + split - 1) / split;
    p.nsplit = p.ksteps > 0 ? (steps + p.ksteps - 1) / p.ksteps : 1;   // no empty split
    p.partial_floats = p.nsplit > 1 ? (size_t)p.nsplit * j.m * ntot : 0;
    return p;
}

void launch_gemm(const GemmJob& j, float* ws, size_t ws_floats, hipStream_t st) {
    launch_gemm_planned(j, gemm_plan(j, ws ? ws_floats : 0), ws, st);
}

void launch_gemm_planned(const GemmJob& j, const GemmPlan& plan, float* ws, hipStream_t st) {
    L3P_REQUIRE(gemm_mfma_supported(j.type), L3P_E_UNSUPPORTED, "gemm: type %d has no MFMA path", j.type);
    L3P_REQUIRE(plan.nsplit == 1 || ws, L3P_E_INVALID, "gemm: split-K plan without a workspace");
    L3P_REQUIRE(j.k % 32 == 0 && j.ldx % 4 == 0 && ((uintptr_t)j.x & 15) == 0, L3P_E_INVALID,
                "gemm: x rows must be 16-byte aligned");
    L3P_REQUIRE(j.m <= 65535 * kBM, L3P_E_INVALID, "gemm: batch %d too large", j.m);
    L3P_REQUIRE(j.nseg >= 1 && j.nseg <= 3, L3P_E_INVALID, "gemm: %d segments", j.nseg);
    GemmArgs a{};
    a.nseg = 0;
    int tiles = 0, ntot = 0;
    for (int i = 0; i < j.nseg; ++i) {
        if (j.seg[i].n == 0) continue;
        a.w[a.nseg] = j.seg[i].w;
        a.y[a.nseg] = j.seg[i].y;
        a.ldy[a.nseg] = j.seg[i].ldy;
        a.n[a.nseg] = j.seg[i].n;
        a.noff[a.nseg] = ntot;
        a.tbeg[a.nseg] = tiles;
        tiles += (j.seg[i].n + plan.bn - 1) / plan.bn;
        ntot += j.seg[i].n;
        ++a.nseg;
    }
    if (j.m == 0 || a.nseg == 0) return;
    a.tbeg[a.nseg] = tiles;
    a.rb = type_row_bytes(j.type, j.k);
    a.k = j.k;
    a.m = j.m;
    a.x = j.x;
    a.ldx = j.ldx;
    a.add = j.add ? 1 : 0;
    a.ntot = ntot;
    a.ksteps = plan.ksteps;
    a.nsplit = plan.nsplit;
    a.streamk = plan.streamk;
    a.kst = plan.ksteps;
    a.bn = plan.bn;
    a.part = (a.nsplit > 1 || a.streamk) ? ws : nullptr;
    L3P_REQUIRE(!a.streamk || ws, L3P_E_INVALID, "gemm: stream-K plan without a workspace");
    switch (j.type) {
    case L3P_Q8_0: launch_typed<L3P_Q8_0>(a, plan.bn, st); break;
    case L3P_Q2_K: launch_typed<L3P_Q2_K>(a, plan.bn, st); break;
    case L3P_Q3_K: launch_typed<L3P_Q3_K>(a, plan.bn, st); break;
    case L3P_Q4_K: launch_typed<L3P_Q4_K>(a, plan.bn, st); break;
    case L3P_Q5_K: launch_typed<L3P_Q5_K>(a, plan.bn, st); break;
    case L3P_Q6_K: launch_typed<L3P_Q6_K>(a, plan.bn, st); break;
    case L3P_F16: launch_typed<L3P_F16>(a, plan.bn, st); break;
    case L3P_F32: launch_typed<L3P_F32>(a, plan.bn, st); break;
    default: launch_typed<L3P_BF16>(a, plan.bn, st); break;
    }
    if (a.nsplit > 1 || a.streamk) {
        bool vec = ntot % 4 == 0;
        for (int i = 0; i < a.nseg; ++i)
            vec = vec && a.n[i] % 4 == 0 && a.ldy[i] % 4 == 0 && ((uintptr_t)a.y[i] & 15) == 0;
        if (vec) launch_kernel(gemm_reduce_kernel<4>, dim3((ntot / 4 + 255) / 256, j.m), dim3(256), 0u, st, a);
        else launch_kernel(gemm_reduce_kernel<1>, dim3((ntot + 255) / 256, j.m), dim3(256), 0u, st, a);
    }
}

// ---------------------------------------------------------------------------
// The Q8_0-activation types (Q4_0, Q4_1, Q5_0, Q5_1, IQ4_NL) on the int8
// matrix cores.  The reference's batched dot for them (matmul_quantized_batch,
// c:2305-2318, with vec_dot_*_q8_0, c:1625-1720) quantizes each activation row
// to Q8_0 and sums, block by block in order,
//   sum += dw * dx * (float)isum  (+ mw * dx * (float)xsum for Q4_1, Q5_1)
// with isum the exact integer dot of the block's weight codes and activation
// quants.  Here q8_rows_kernel quantizes the rows once (int8 quants, the fp16
// scale as float, the quant sum), a workgroup expands a 64 x 64 weight tile to
// int8 codes in LDS (Q4_0 and Q5_0 subtract their offset 8 or 16 byte-wise,
// IQ4_NL maps its nibbles through a byte permute of its table), and one
// v_mfma_i32_16x16x32_i8 gives the exact isum of one block for 16 x 16
// outputs.  Each output's lane then adds the block terms in block order with
// the reference's expression, so no K split and no reordering of the terms.
// ---------------------------------------------------------------------------
namespace {

__global__ void __launch_bounds__(256) q8_rows_kernel(const float* __restrict__ x, int ldx, int k, int rows,
                                                      int8_t* __restrict__ xq, float* __restrict__ dx,
                                                      float* __restrict__ sx) {
    const int nb = k >> 5;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * nb) return;
    const int r = (int)(i / nb), b = (int)(i % nb);
    const float4* src = reinterpret_cast<const float4*>(x + (size_t)r * ldx + 32 * b);
    float v[32];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const float4 f = src[u];
        v[4 * u] = f.x;
        v[4 * u + 1] = f.y;
        v[4 * u + 2] = f.z;
        v[4 * u + 3] = f.w;
    }
    QBlock q;
    quantize32(v, q);   // quantize_row_q8_0 (c:1508-1528)
    uint32_t wq[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
        wq[u] = (uint32_t)(uint8_t)q.q[4 * u] | ((uint32_t)(uint8_t)q.q[4 * u + 1] << 8) |
                ((uint32_t)(uint8_t)q.q[4 * u + 2] << 16) | ((uint32_t)(uint8_t)q.q[4 * u + 3] << 24);
    uint4* dst = reinterpret_cast<uint4*>(xq + (size_t)r * k + 32 * b);
    dst[0] = make_uint4(wq[0], wq[1], wq[2], wq[3]);
    dst[1] = make_uint4(wq[4], wq[5], wq[6], wq[7]);
    dx[i] = h2f_exact(q.dh);   // fp16_to_fp32(xq.d)
    sx[i] = (float)q.sum;
}

// One thread's 16 weight codes of a step: row t / 4 of the tile, elements
// e0 .. e0 + 15 (half of a 32-element block), fetched one step ahead.
struct Q8aRegs {
    uint4 x;            // 16 activation quants
    uint4 q;            // the block's 16 nibble-pair bytes
    uint32_t h0, h1;    // d (| m << 16), the 32 high bits (Q5_0, Q5_1)
    float dxv, sxv;     // one activation block's scale and quant sum
};

template <int QT>
__device__ __forceinline__ void fetch_q8a_w(Q8aRegs& r, const uint8_t* row, int e0) {
    if constexpr (QT == L3P_Q4_0 || QT == L3P_IQ4_NL) {   // 18 bytes: d, qs[16]
        const uint8_t* b = row + (size_t)(e0 >> 5) * 18;
        r.h0 = *reinterpret_cast<const uint16_t*>(b);
        __builtin_memcpy(&r.q, b + 2, 16);
    } else if constexpr (QT == L3P_Q4_1) {   // 20 bytes: d, m, qs[16]
        const uint8_t* b = row + (size_t)(e0 >> 5) * 20;
        __builtin_memcpy(&r.h0, b, 4);
        __builtin_memcpy(&r.q, b + 4, 16);
    } else if constexpr (QT == L3P_Q5_0) {   // 22 bytes: d, qh[4], qs[16]
        const uint8_t* b = row + (size_t)(e0 >> 5) * 22;
        r.h0 = *reinterpret_cast<const uint16_t*>(b);
        __builtin_memcpy(&r.h1, b + 2, 4);
        __builtin_memcpy(&r.q, b + 6, 16);
    } else {   // Q5_1, 24 bytes: d, m, qh[4], qs[16]
        const uint8_t* b = row + (size_t)(e0 >> 5) * 24;
        __builtin_memcpy(&r.h0, b, 4);
        __builtin_memcpy(&r.h1, b + 4, 4);
        __builtin_memcpy(&r.q, b + 8, 16);
    }
}

// IQ4_NL's values (kvalues_iq4nl, c:920-934) of the four nibbles in the bytes
// of nb: byte permutes over the table's two halves and a byte select on bit 3.
__device__ __forceinline__ uint32_t iq4nl_bytes(uint32_t nb) {
    const uint32_t sel = nb & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(0xF6EADDCFu, 0xBFAD9881u, sel);   // -127 -104 -83 -65 -49 -35 -22 -10
    const uint32_t hi = __builtin_amdgcn_perm(0x71594535u, 0x26190D01u, sel);   // 1 13 25 38 53 69 89 113
    const uint32_t m = ((nb >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// byte-wise x - c for bytes x in 0..31 and c <= 16, as int8 (no borrow
// crosses a byte: x | 0x80 - c stays >= 0x70)
__device__ __forceinline__ uint32_t sub_bytes(uint32_t x, uint32_t c4) { return ((x | 0x80808080u) - c4) ^ 0x80808080u; }

// the 16 int8 codes of elements e0 .. e0 + 15 (the weight values over d; the
// codes vec_dot_*_q8_0 multiplies with the activation quants)
template <int QT>
__device__ __forceinline__ uint4 decode_q8a_w(const Q8aRegs& r, int e0) {
    const int hi = (e0 >> 4) & 1;   // elements 16..31: the high nibbles
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    uint32_t o[4];
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
        uint32_t nb = (qw[w4] >> (4 * hi)) & 0x0f0f0f0fu;
        if constexpr (QT == L3P_Q5_0 || QT == L3P_Q5_1) {
            // bits 16 hi + 4 w4 .. + 3 of qh to bit 4 of the four bytes
            const uint32_t hb = (r.h1 >> (16 * hi + 4 * w4)) & 0xfu;
            nb |= ((hb * 0x00204081u) & 0x01010101u) << 4;
        }
        if constexpr (QT == L3P_Q4_0) o[w4] = sub_bytes(nb, 0x08080808u);
        else if constexpr (QT == L3P_Q5_0) o[w4] = sub_bytes(nb, 0x10101010u);
        else if constexpr (QT == L3P_IQ4_NL) o[w4] = iq4nl_bytes(nb);
        else o[w4] = nb;   // Q4_1, Q5_1: codes 0..15, 0..31
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

constexpr int kQLD = 80;   // LDS row stride of the int8 tiles (bytes, 16-byte aligned rows)

template <int QT>
__global__ void __launch_bounds__(256) gemm_q8a_kernel(GemmArgs a, const int8_t* __restrict__ xq,
                                                       const float* __restrict__ dxg, const float* __restrict__ sxg) {
    constexpr bool kMin = QT == L3P_Q4_1 || QT == L3P_Q5_1;
    __shared__ __align__(16) int8_t xs[kBM * kQLD];
    __shared__ __align__(16) int8_t ws[64 * kQLD];
    __shared__ __align__(16) float dxs[2][kBM];   // activation block scales [block of the step][row]
    __shared__ __align__(16) float sxs[2][kBM];   // activation quant sums
    __shared__ __align__(16) float dws[2][64];    // weight block scales [block][weight row]
    __shared__ __align__(16) float mws[2][64];    // weight block minima
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wm = w >> 1, wn = w & 1;       // this wave's 32 x 32 block of the 64 x 64 tile
    const int g = lane >> 4, i16 = lane & 15;
    const TileRef tr = tile_ref<64>(a, blockIdx.x, blockIdx.y);
    const int nb = a.k >> 5;
    float acc[2][2][4];
#pragma unroll
    for (int im = 0; im < 2; ++im)
#pragma unroll
        for (int in = 0; in < 2; ++in)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[im][in][r] = 0.0f;
    Q8aRegs R;
    auto fetch = [&](int k0) {
        const int m = tr.m0 + (t >> 2), kx = k0 + 16 * (t & 3);
        R.x = make_uint4(0u, 0u, 0u, 0u);
        if (m < a.m && kx < a.k) R.x = *reinterpret_cast<const uint4*>(xq + (size_t)m * a.k + kx);
        R.dxv = 0.0f;
        R.sxv = 0.0f;
        if (t < 2 * kBM) {   // scale and quant sum of row t % 64, block t / 64 of the step
            const int mm = tr.m0 + (t & 63), kb = (k0 >> 5) + (t >> 6);
            if (mm < a.m && kb < nb) {
                R.dxv = dxg[(size_t)mm * nb + kb];
                if (kMin) R.sxv = sxg[(size_t)mm * nb + kb];
            }
        }
        const int n = tr.n0 + (t >> 2);
        R.q = make_uint4(0u, 0u, 0u, 0u);
        R.h0 = R.h1 = 0u;
        if (n < tr.N && kx < a.k) fetch_q8a_w<QT>(R, tr.W + (size_t)n * a.rb, kx);
    };
    fetch(0);
    for (int k0 = 0; k0 < a.k; k0 += kBK) {
        const int kx = k0 + 16 * (t & 3);
        *reinterpret_cast<uint4*>(xs + (t >> 2) * kQLD + 16 * (t & 3)) = R.x;
        *reinterpret_cast<uint4*>(ws + (t >> 2) * kQLD + 16 * (t & 3)) = decode_q8a_w<QT>(R, kx);
        if (t < 2 * kBM) {
            dxs[t >> 6][t & 63] = R.dxv;
            if (kMin) sxs[t >> 6][t & 63] = R.sxv;
        }
        if ((t & 1) == 0) {   // the block's d (and m) of row t / 4, block (t / 2) % 2
            dws[(t >> 1) & 1][t >> 2] = h2f_exact(R.h0 & 0xffffu);
            if (kMin) mws[(t >> 1) & 1][t >> 2] = h2f_exact(R.h0 >> 16);
        }
        __syncthreads();
        if (k0 + kBK < a.k) fetch(k0 + kBK);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            if (k0 + 32 * kb >= a.k) break;
            long af[2], bf[2];
#pragma unroll
            for (int im = 0; im < 2; ++im)
                af[im] = *reinterpret_cast<const long*>(xs + (32 * wm + 16 * im + i16) * kQLD + 32 * kb + 8 * g);
#pragma unroll
            for (int in = 0; in < 2; ++in)
                bf[in] = *reinterpret_cast<const long*>(ws + (32 * wn + 16 * in + i16) * kQLD + 32 * kb + 8 * g);
#pragma unroll
            for (int in = 0; in < 2; ++in) {
                const float dw = dws[kb][32 * wn + 16 * in + i16];
                const float mw = kMin ? mws[kb][32 * wn + 16 * in + i16] : 0.0f;
#pragma unroll
                for (int im = 0; im < 2; ++im) {
                    // D lane (g, i16): rows (activation rows) 4 g .. 4 g + 3 of column i16 (weight row)
                    const int32x4 is = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[im], bf[in], int32x4{0, 0, 0, 0}, 0, 0, 0);
                    const float4 dx4 = *reinterpret_cast<const float4*>(&dxs[kb][32 * wm + 16 * im + 4 * g]);
                    const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
                    float sxr[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    if (kMin) {
                        const float4 s4 = *reinterpret_cast<const float4*>(&sxs[kb][32 * wm + 16 * im + 4 * g]);
                        sxr[0] = s4.x;
                        sxr[1] = s4.y;
                        sxr[2] = s4.z;
                        sxr[3] = s4.w;
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float term = dw * dxr[r] * (float)is[r];
                        if (kMin) term = term + mw * dxr[r] * sxr[r];
                        acc[im][in][r] += term;
                    }
                }
            }
        }
        __syncthreads();
    }
    float* const Y = a.y[tr.sg];
    const int ldy = a.ldy[tr.sg];
#pragma unroll
    for (int im = 0; im < 2; ++im)
#pragma unroll
        for (int in = 0; in < 2; ++in) {
            const int n = tr.n0 + 32 * wn + 16 * in + i16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = tr.m0 + 32 * wm + 16 * im + 4 * g + r;
                if (m < a.m && n < tr.N) {
                    float* p = Y + (size_t)m * ldy + n;
                    *p = a.add ? *p + acc[im][in][r] : acc[im][in][r];
                }
            }
        }
}

}  // namespace

bool gemm_q8_activation(int type) {
    return type == L3P_Q4_0 || type == L3P_Q4_1 || type == L3P_Q5_0 || type == L3P_Q5_1 || type == L3P_IQ4_NL;
}

size_t gemm_q8a_ws_floats(int rows, int k) {
    // int8 quants (k bytes a row) and two floats per block, 256-byte aligned parts
    const size_t q = ((size_t)rows * k + 255) / 256 * 64;
    const size_t s = ((size_t)rows * (k / 32) + 63) / 64 * 64;
    return q + 2 * s;
}

void launch_gemm_q8a(const GemmJob& j, float* ws, size_t ws_floats, hipStream_t st) {
    L3P_REQUIRE(gemm_q8_activation(j.type), L3P_E_UNSUPPORTED, "gemm: type %d has no int8 path", j.type);
    L3P_REQUIRE(j.k % 32 == 0 && j.ldx % 4 == 0 && ((uintptr_t)j.x & 15) == 0, L3P_E_INVALID,
                "gemm: x rows must be 16-byte aligned");
    L3P_REQUIRE(j.nseg >= 1 && j.nseg <= 3, L3P_E_INVALID, "gemm: %d segments", j.nseg);
    if (j.m == 0) return;
    // rows per launch: as many as the workspace holds the quantized rows of
    const size_t per_row = gemm_q8a_ws_floats(1, j.k);
    L3P_REQUIRE(ws && ws_floats >= gemm_q8a_ws_floats(1, j.k), L3P_E_INVALID, "gemm: workspace of %zu floats",
                ws_floats);
    int cr = (int)std::min<size_t>((size_t)j.m, ws_floats / per_row);
    while (cr > 1 && gemm_q8a_ws_floats(cr, j.k) > ws_floats) --cr;
    cr = std::min(cr, 65535 * kBM);
    GemmArgs a{};
    int tiles = 0;
    for (int i = 0; i < j.nseg; ++i) {
        if (j.seg[i].n == 0) continue;
        a.w[a.nseg] = j.seg[i].w;
        a.y[a.nseg] = j.seg[i].y;
        a.ldy[a.nseg] = j.seg[i].ldy;
        a.n[a.nseg] = j.seg[i].n;
        a.tbeg[a.nseg] = tiles;
        tiles += (j.seg[i].n + 63) / 64;
        ++a.nseg;
    }
    if (a.nseg == 0) return;
    a.tbeg[a.nseg] = tiles;
    a.rb = type_row_bytes(j.type, j.k);
    a.k = j.k;
    a.add = j.add ? 1 : 0;
    a.bn = 64;
    for (int b0 = 0; b0 < j.m; b0 += cr) {
        const int rows = std::min(cr, j.m - b0);
        int8_t* xq = reinterpret_cast<int8_t*>(ws);
        float* dx = ws + ((size_t)rows * j.k + 255) / 256 * 64;
        float* sx = dx + ((size_t)rows * (j.k / 32) + 63) / 64 * 64;
        const int64_t nblk = (int64_t)rows * (j.k / 32);
        launch_kernel(q8_rows_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0u, st,
                      j.x + (size_t)b0 * j.ldx, j.ldx, j.k, rows, xq, dx, sx);
        GemmArgs c = a;
        c.m = rows;
        for (int i = 0; i < c.nseg; ++i) c.y[i] = a.y[i] + (size_t)b0 * a.ldy[i];
        const dim3 grid(tiles, (rows + kBM - 1) / kBM);
        switch (j.type) {
        case L3P_Q4_0: launch_kernel(gemm_q8a_kernel<L3P_Q4_0>, grid, dim3(256), 0u, st, c, xq, dx, sx); break;
        case L3P_Q4_1: launch_kernel(gemm_q8a_kernel<L3P_Q4_1>, grid, dim3(256), 0u, st, c, xq, dx, sx); break;
        case L3P_Q5_0: launch_kernel(gemm_q8a_kernel<L3P_Q5_0>, grid, dim3(256), 0u, st, c, xq, dx, sx); break;
        case L3P_Q5_1: launch_kernel(gemm_q8a_kernel<L3P_Q5_1>, grid, dim3(256), 0u, st, c, xq, dx, sx); break;
        default: launch_kernel(gemm_q8a_kernel<L3P_IQ4_NL>, grid, dim3(256), 0u, st, c, xq, dx, sx); break;
        }
    }
}

// ---------------------------------------------------------------------------
// The split-K partials of l3p_gemm_static: a file-scope device array instead
// of a context workspace, so that entry point allocates nothing.  Each GPU
// holds its own copy for the life of the process; host code uses the device
// address that hipGetSymbolAddress returns for the current device (the
// array's name is only a host-side stand-in).  Calls that overlap on one GPU
// share it and race.
// ---------------------------------------------------------------------------
namespace {
__device__ __align__(256) float scratch[kGemmStaticScratchFloats];
constexpr int kMaxDevices = 64;
}  // namespace

float* gemm_static_scratch() {
    static std::mutex mu;
    static float* ptr[kMaxDevices] = {};
    int dev = 0;
    L3P_HIP(hipGetDevice(&dev));
    L3P_REQUIRE(dev >= 0 && dev < kMaxDevices, L3P_E_UNSUPPORTED, "gemm_static: device %d", dev);
    std::lock_guard<std::mutex> g(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        L3P_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        ptr[dev] = static_cast<float*>(p);
    }
    return ptr[dev];
}
