// gemv2.hip — streaming decode GEMVs for Q8_0 and Q4_0 blocks (gfx950).
//
// Persistent workgroups walk row tiles of the matrix.  A tile (R consecutive
// rows, contiguous in HBM) is copied into LDS with global_load_lds_dwordx4
// (HBM -> LDS without passing through VGPRs); the next tile's copy is issued
// before the current tile is reduced, so it is in flight during the compute.
//
// Thread t owns block column col(t) for the whole kernel and keeps that
// block's activation in registers.  Q8_0 (34 B) and Q4_0 (18 B) blocks start
// 2 bytes into a dword for odd columns, so even columns go to even waves and
// odd columns to odd waves: realignment is then wave-uniform (one
// v_alignbyte per dword for even waves, nothing for odd ones).
//
// Inner products are integer dot4 (v_dot4_i32_i8):
//   Q4_0: against the Q8_0 quantized activation, exactly as the reference's
//         vec_dot_q4_0_q8_0 (c:1625-1643);
//   Q8_0: against x decomposed per 32-block into four int8 digits,
//         x = 2^(e-6) (d0 + d1/2^7 + d2/2^14 + d3/2^21), which keeps every
//         value to 2^-27 of its block maximum; the four integer block dots
//         are exact and are combined in fp32 (the reference multiplies the
//         exactly dequantized weights with fp32 x, c:2136-2176).
// Row partials are reduced across the wave by a transpose-reduce, then across
// waves in a fixed order, so results are deterministic.
#include "device_common.h"
#include "internal.h"

#include <map>
#include <mutex>
#include <tuple>

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBufs = 3;          // tiles resident in LDS: one computed, two in flight
constexpr int kMaxOut = 2048;     // per-workgroup result slots kept in LDS

using namespace l3pd;

// HBM -> LDS copy of one tile.  Wave w copies the contiguous byte range
// [w*S, (w+1)*S) of the tile (S = per-wave share rounded up to 16 bytes) with
// global_load_lds_dwordx4; lane i of an instruction lands at that
// instruction's LDS base + 16 i.  Returns the number of copy instructions the
// wave issued, which is what the wave later waits on.  Weights are read once
// per call, so the copies are non-temporal (cache policy nt).
__device__ __forceinline__ int tile_dma(uint32_t* dst, const uint8_t* __restrict__ src, int nbytes, int w, int nw,
                                        int lane) {
    const int S = ((nbytes + nw - 1) / nw + 15) & ~15;
    const int lo = w * S;
    const int hi = min(nbytes, lo + S);
    int n = 0;
    for (int off = lo; off < hi; off += 1024, ++n) {
        const int o = off + lane * 16;
        if (o < hi) __builtin_amdgcn_global_load_lds(src + o, (lds_void*)(dst + (off >> 2)), 16, 0, 2);
    }
    return n;
}

// Workgroup barrier for LDS traffic only.  __syncthreads() carries a release
// fence that waits for every outstanding memory operation (vmcnt(0)), which
// would also wait for the tile copies kept in flight.
__device__ __forceinline__ void lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until at most n of this wave's vector-memory operations are
// outstanding (vmcnt takes an immediate; n is small and wave-uniform).
__device__ __forceinline__ void wait_vm(int n) {
    n = __builtin_amdgcn_readfirstlane(n);
    // s_waitcnt encoding on gfx9: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
#define L3P_W(k) case k: __builtin_amdgcn_s_waitcnt((k & 15) | ((k >> 4) << 14) | (7 << 4) | (15 << 8)); break;
    switch (n) {
        L3P_W(0) L3P_W(1) L3P_W(2) L3P_W(3) L3P_W(4) L3P_W(5) L3P_W(6) L3P_W(7)
        L3P_W(8) L3P_W(9) L3P_W(10) L3P_W(11) L3P_W(12) L3P_W(13) L3P_W(14) L3P_W(15)
        L3P_W(16) L3P_W(17) L3P_W(18) L3P_W(19) L3P_W(20) L3P_W(21) L3P_W(22) L3P_W(23)
        default: __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); break;   // vmcnt(0)
    }
#undef L3P_W
}

// Reduce N per-thread row partials over a wave: after the call every lane in
// group g (64/N consecutive lanes) holds the wave total of row rowof<N>(lane).
template <int N>
__device__ __forceinline__ constexpr int log2c() {
    return N >= 16 ? 4 : N >= 8 ? 3 : N >= 4 ? 2 : N >= 2 ? 1 : 0;
}
template <int N>
__device__ __forceinline__ int rowof(int lane) {
    constexpr int L = log2c<N>();
    int r = 0;
#pragma unroll
    for (int s = 0; s < L; ++s) r |= ((lane >> (5 - s)) & 1) << (L - 1 - s);
    return r;
}
template <int N>
__device__ __forceinline__ float xreduce(float (&v)[N], int lane) {
    constexpr int L = log2c<N>();
#pragma unroll
    for (int s = 0; s < L; ++s) {
        const int m = 32 >> s;
        const bool up = (lane & m) != 0;
        const int half = N >> (s + 1);
#pragma unroll
        for (int i = 0; i < (N >> 1); ++i) {
            if (i < half) {
                const float send = up ? v[i] : v[i + half];
                const float keep = up ? v[i + half] : v[i];
                v[i] = keep + __shfl_xor(send, m, 64);
            }
        }
    }
    float r = v[0];
#pragma unroll
    for (int m = 32 >> L; m > 0; m >>= 1) r += __shfl_xor(r, m, 64);
    return r;
}

struct TileLoc {
    int seg, r0, nr;
};
template <int R, bool PAIR>
__device__ __forceinline__ TileLoc locate_tile(const GemvBatch& B, int tile) {
    int s = 0;
    if (!PAIR) {
        while (s < B.nseg - 1) {
            const int nt = (B.seg[s].rows + R - 1) / R;
            if (tile < nt) break;
            tile -= nt;
            ++s;
        }
    }
    TileLoc L;
    L.seg = s;
    L.r0 = tile * R;
    L.nr = min(R, B.seg[s].rows - L.r0);
    return L;
}

template <int R, bool PAIR>
__device__ __forceinline__ int issue_tile(const GemvBatch& B, int tile, uint32_t* buf, uint32_t rb, int w, int nw,
                                          int lane) {
    const TileLoc L = locate_tile<R, PAIR>(B, tile);
    int n = tile_dma(buf, B.seg[L.seg].w + (size_t)L.r0 * rb, L.nr * (int)rb, w, nw, lane);
    if (PAIR) n += tile_dma(buf + (R * rb >> 2), B.seg[1].w + (size_t)L.r0 * rb, L.nr * (int)rb, w, nw, lane);
    return n;
}

// Cross-wave sum of the per-wave row totals and the epilogue.  The row
// results are kept in LDS (out_lds[k*R + r] for the workgroup's k-th tile)
// and written to HBM after the last tile: on gfx9 a wait for outstanding
// loads also waits for every outstanding store, so stores inside the loop
// would add a memory round trip to every tile.
template <int R, bool PAIR>
__device__ __forceinline__ void finish_tile(const GemvBatch& B, const TileLoc& L, float (&acc)[PAIR ? 2 * R : R],
                                            float* red, float* out_lds, int k, int w, int nw, int lane) {
    constexpr int NRR = PAIR ? 2 * R : R;
    const float tot = xreduce<NRR>(acc, lane);
    if ((lane & ((64 / NRR) - 1)) == 0) red[w * NRR + rowof<NRR>(lane)] = tot;
    lds_sync();
    const int t = threadIdx.x;
    if (t < L.nr) {
        float a = 0.0f, b = 0.0f;
        for (int j = 0; j < nw; ++j) {
            a += red[j * NRR + t];
            if (PAIR) b += red[j * NRR + R + t];
        }
        out_lds[k * R + t] = PAIR ? (B.epilogue == EPI_GEGLU ? ref_geglu(a, b) : ref_swiglu(a, b)) : a;
    }
}

// Write the workgroup's results: tile k of the workgroup is global tile
// blockIdx.x + k*gridDim.x.
template <int R, bool PAIR>
__device__ __forceinline__ void flush_results(const GemvBatch& B, const float* out_lds, int ntiles) {
    const int nk = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    for (int j = threadIdx.x; j < nk * R; j += blockDim.x) {
        const int k = j / R, r = j % R;
        const TileLoc L = locate_tile<R, PAIR>(B, blockIdx.x + k * gridDim.x);
        if (r >= L.nr) continue;
        float* y = (PAIR ? B.seg[0].y : B.seg[L.seg].y) + L.r0 + r;
        if (!PAIR && B.epilogue == EPI_ADD) *y += out_lds[j];
        else *y = out_lds[j];
    }
}

__device__ __forceinline__ int col_of(int t) {
    const int w = t >> 6, lane = t & 63;
    return 2 * (64 * (w >> 1) + lane) + (w & 1);
}

// ---------------------------------------------------------------------------
// Q8_0 x digit form
// ---------------------------------------------------------------------------
template <int R, bool PAIR>
__global__ void __launch_bounds__(1024) gemv2_q8_0(GemvBatch B, int cols, XDig xd, int ntiles) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int NRR = PAIR ? 2 * R : R;
    const int nb = cols >> 5;
    const uint32_t rb = (uint32_t)nb * 34u;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, nw = blockDim.x >> 6;
    const uint32_t tile_dw = ((PAIR ? 2 : 1) * R * rb + 15) / 16 * 4;
    float* red = reinterpret_cast<float*>(lds + kBufs * tile_dw);
    float* out_lds = red + nw * NRR;

    // prologue: the first kBufs-1 tiles in flight
    int cnt[kBufs];
#pragma unroll
    for (int b = 0; b < kBufs; ++b) cnt[b] = 0;
#pragma unroll
    for (int b = 0; b < kBufs - 1; ++b) {
        const int tb = blockIdx.x + b * gridDim.x;
        if (tb < ntiles) cnt[b] = issue_tile<R, PAIR>(B, tb, lds + b * tile_dw, rb, w, nw, lane);
    }

    const int col = col_of(t);
    const bool active = col < nb;
    const bool odd = (w & 1) != 0;
    int xw[4][8];
    float xs = 0.0f;
    if (active) {
        const int4* p = reinterpret_cast<const int4*>(xd.dg + 128 * col);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int4 a = p[2 * k], b = p[2 * k + 1];
            xw[k][0] = a.x; xw[k][1] = a.y; xw[k][2] = a.z; xw[k][3] = a.w;
            xw[k][4] = b.x; xw[k][5] = b.y; xw[k][6] = b.z; xw[k][7] = b.w;
        }
        xs = xd.s[col];
    }

    int k = 0;
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x, ++k) {
        const TileLoc L = locate_tile<R, PAIR>(B, tile);
        // wait for this tile's copy; the next kBufs-2 stay in flight
        int newer = 0;
#pragma unroll
        for (int b = 1; b < kBufs - 1; ++b) newer += cnt[(k + b) % kBufs];
        wait_vm(newer);
        lds_sync();
        {
            const int tn = tile + (kBufs - 1) * gridDim.x;
            const int bn = (k + kBufs - 1) % kBufs;
            cnt[bn] = tn < ntiles ? issue_tile<R, PAIR>(B, tn, lds + bn * tile_dw, rb, w, nw, lane) : 0;
        }
        const uint32_t cur = (uint32_t)(k % kBufs) * tile_dw;   // LDS dword offset of this tile
        float acc[NRR];
#pragma unroll
        for (int i = 0; i < NRR; ++i) {
            float a = 0.0f;
            if (active && (i % R) < L.nr) {
                const uint32_t E = ((uint32_t)i * rb + 34u * (uint32_t)col) >> 2;
                uint32_t dw[9];
#pragma unroll
                for (int k = 0; k < 9; ++k) dw[k] = lds[cur + E + k];
                uint32_t q[8];
                float d;
                if (odd) {
                    d = h2f(dw[0] >> 16);
#pragma unroll
                    for (int k = 0; k < 8; ++k) q[k] = dw[k + 1];
                } else {
                    d = h2f(dw[0]);
#pragma unroll
                    for (int k = 0; k < 8; ++k) q[k] = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2);
                }
                int I[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    int s = 0;
#pragma unroll
                    for (int k = 0; k < 8; ++k) s = __builtin_amdgcn_sdot4((int)q[k], xw[g][k], s, false);
                    I[g] = s;
                }
                const float c7 = 0.0078125f;
                const float f = (float)I[0] + ((float)I[1] + ((float)I[2] + (float)I[3] * c7) * c7) * c7;
                a = f * (d * xs);
            }
            acc[i] = a;
        }
        finish_tile<R, PAIR>(B, L, acc, red, out_lds, k, w, nw, lane);
        lds_sync();
    }
    flush_results<R, PAIR>(B, out_lds, ntiles);
}

// ---------------------------------------------------------------------------
// Q4_0 against the Q8_0 activation (vec_dot_q4_0_q8_0, c:1625-1643)
// ---------------------------------------------------------------------------
template <int R, bool PAIR>
__global__ void __launch_bounds__(1024) gemv2_q4_0(GemvBatch B, int cols, XQ8 xq, int ntiles) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int NRR = PAIR ? 2 * R : R;
    const int nb = cols >> 5;
    const uint32_t rb = (uint32_t)nb * 18u;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, nw = blockDim.x >> 6;
    const uint32_t tile_dw = ((PAIR ? 2 : 1) * R * rb + 15) / 16 * 4;
    float* red = reinterpret_cast<float*>(lds + kBufs * tile_dw);
    float* out_lds = red + nw * NRR;

    // prologue: the first kBufs-1 tiles in flight
    int cnt[kBufs];
#pragma unroll
    for (int b = 0; b < kBufs; ++b) cnt[b] = 0;
#pragma unroll
    for (int b = 0; b < kBufs - 1; ++b) {
        const int tb = blockIdx.x + b * gridDim.x;
        if (tb < ntiles) cnt[b] = issue_tile<R, PAIR>(B, tb, lds + b * tile_dw, rb, w, nw, lane);
    }

    const int col = col_of(t);
    const bool active = col < nb;
    const bool odd = (w & 1) != 0;
    int xw[8];
    float dx = 0.0f;
    int xsum8 = 0;
    if (active) {
        const int4* p = reinterpret_cast<const int4*>(xq.qs + 32 * col);
        const int4 a = p[0], b = p[1];
        xw[0] = a.x; xw[1] = a.y; xw[2] = a.z; xw[3] = a.w;
        xw[4] = b.x; xw[5] = b.y; xw[6] = b.z; xw[7] = b.w;
        dx = xq.d[col];
        xsum8 = 8 * xq.sum[col];
    }

    int k = 0;
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x, ++k) {
        const TileLoc L = locate_tile<R, PAIR>(B, tile);
        // wait for this tile's copy; the next kBufs-2 stay in flight
        int newer = 0;
#pragma unroll
        for (int b = 1; b < kBufs - 1; ++b) newer += cnt[(k + b) % kBufs];
        wait_vm(newer);
        lds_sync();
        {
            const int tn = tile + (kBufs - 1) * gridDim.x;
            const int bn = (k + kBufs - 1) % kBufs;
            cnt[bn] = tn < ntiles ? issue_tile<R, PAIR>(B, tn, lds + bn * tile_dw, rb, w, nw, lane) : 0;
        }
        const uint32_t cur = (uint32_t)(k % kBufs) * tile_dw;   // LDS dword offset of this tile
        float acc[NRR];
#pragma unroll
        for (int i = 0; i < NRR; ++i) {
            float a = 0.0f;
            if (active && (i % R) < L.nr) {
                const uint32_t E = ((uint32_t)i * rb + 18u * (uint32_t)col) >> 2;
                uint32_t dw[5];
#pragma unroll
                for (int k = 0; k < 5; ++k) dw[k] = lds[cur + E + k];
                uint32_t q[4];
                float dwt;
                if (odd) {
                    dwt = h2f(dw[0] >> 16);
#pragma unroll
                    for (int k = 0; k < 4; ++k) q[k] = dw[k + 1];
                } else {
                    dwt = h2f(dw[0]);
#pragma unroll
                    for (int k = 0; k < 4; ++k) q[k] = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2);
                }
                int isum = -xsum8;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    isum = __builtin_amdgcn_sdot4((int)(q[k] & 0x0f0f0f0fu), xw[k], isum, false);
                    isum = __builtin_amdgcn_sdot4((int)((q[k] >> 4) & 0x0f0f0f0fu), xw[4 + k], isum, false);
                }
                a = dwt * dx * (float)isum;
            }
            acc[i] = a;
        }
        finish_tile<R, PAIR>(B, L, acc, red, out_lds, k, w, nw, lane);
        lds_sync();
    }
    flush_results<R, PAIR>(B, out_lds, ntiles);
}

// ---------------------------------------------------------------------------
// x -> four int8 digits per element with a power-of-two scale per 32-block.
// X = x * 2^(6-e) with amax < 2^e, so |X| < 64; each digit is the nearest
// integer to the scaled remainder, every step exact in fp32.
// ---------------------------------------------------------------------------
__global__ void x_digits_kernel(const float* __restrict__ x, int nb, XDig out) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = x[32 * b + j];
    int8_t dg[4][32];
    const float sc = digits32(v, dg);
    int4* dst = reinterpret_cast<int4*>(out.dg + 128 * b);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int* p = reinterpret_cast<const int*>(dg[k]);
        dst[2 * k] = make_int4(p[0], p[1], p[2], p[3]);
        dst[2 * k + 1] = make_int4(p[4], p[5], p[6], p[7]);
    }
    out.s[b] = sc;
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------
int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 0;
        if (cus <= 0) cus = 256;
    }
    return cus;
}

int tile_budget() {
    static int kb = -1;
    if (kb < 0) {
        const char* e = getenv("L3P_GEMV_TILE_KB");
        kb = e ? atoi(e) : 12;
        if (kb < 4) kb = 4;
    }
    return kb * 1024;
}

template <typename K>
int occupancy(K kern, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, size_t>, int> cache;
    std::lock_guard<std::mutex> g(mu);
    auto key = std::make_tuple((const void*)kern, threads, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    if (lds > 65536)
        L3P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int n = 0;
    L3P_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds));
    if (n < 1) n = 1;
    cache[key] = n;
    return n;
}

template <int R, bool PAIR>
void launch2(int type, const GemvBatch& b, int cols, const XPrep& x, hipStream_t st) {
    const int nb = cols / 32;
    const uint32_t rb = (uint32_t)type_row_bytes(type, cols);
    const int threads = (nb + 127) / 128 * 128;
    const size_t tile = ((size_t)(PAIR ? 2 : 1) * R * rb + 15) / 16 * 16;
    int tiles = 0;
    if (PAIR) tiles = (b.seg[0].rows + R - 1) / R;
    else
        for (int s = 0; s < b.nseg; ++s) tiles += (b.seg[s].rows + R - 1) / R;
    if (tiles == 0) return;
    // result slots: each workgroup keeps R floats per tile it processes
    auto lds_for = [&](int grid) {
        const int per = (tiles + grid - 1) / grid;
        return kBufs * tile + (size_t)(threads / 64) * (PAIR ? 2 * R : R) * 4 + (size_t)per * R * 4;
    };
    auto run = [&](auto kern, auto xarg) {
        int grid = std::min(tiles, occupancy(kern, threads, lds_for(device_cus())) * device_cus());
        grid = std::max(grid, (tiles * R + kMaxOut - 1) / kMaxOut);
        const size_t lds = lds_for(grid);
        if (lds > 65536)
            L3P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(kern, dim3(grid), dim3(threads), lds, st, b, cols, xarg, tiles);
    };
    if (type == L3P_Q8_0) run(gemv2_q8_0<R, PAIR>, x.dig);
    else run(gemv2_q4_0<R, PAIR>, x.q8);
    L3P_HIP(hipGetLastError());
}

}  // namespace

bool gemv2_supported(int type, int cols) {
    if (type != L3P_Q8_0 && type != L3P_Q4_0) return false;
    return cols > 0 && cols % 256 == 0 && cols / 32 <= 1024;   // rows are 16-byte multiples
}

void launch_gemv2(int type, const GemvBatch& b, int cols, const XPrep& x, hipStream_t st) {
    const size_t rb = type_row_bytes(type, cols);
    const size_t per = (b.pair ? 2 : 1) * rb;
    const size_t budget = (size_t)tile_budget();
    int R = 1;
    while (R < 8 && (size_t)(2 * R) * per <= budget) R *= 2;   // tile of R rows within the budget
    if (b.pair) {
        switch (R) {
        case 8: launch2<8, true>(type, b, cols, x, st); break;
        case 4: launch2<4, true>(type, b, cols, x, st); break;
        case 2: launch2<2, true>(type, b, cols, x, st); break;
        default: launch2<1, true>(type, b, cols, x, st); break;
        }
    } else {
        switch (R) {
        case 8: launch2<8, false>(type, b, cols, x, st); break;
        case 4: launch2<4, false>(type, b, cols, x, st); break;
        case 2: launch2<2, false>(type, b, cols, x, st); break;
        default: launch2<1, false>(type, b, cols, x, st); break;
        }
    }
}

void launch_x_digits(const float* x, int cols, const XDig& xd, hipStream_t st) {
    const int nb = cols / 32;
    hipLaunchKernelGGL(x_digits_kernel, dim3((nb + 127) / 128), dim3(128), 0, st, x, nb, xd);
    L3P_HIP(hipGetLastError());
}
