// gemv4.hip — streaming decode GEMVs for Q8_0 and Q4_0 blocks (gfx950),
// split over 64-block column chunks, with the activation's RMSNorm and its
// integer form computed in the prologue.
//
// Work split.  A row of nb blocks is cut into NC = ceil(nb/64) chunks of 64
// blocks (Q8_0: 2176 B, Q4_0: 1152 B; both 16-byte multiples, so every chunk
// of a row whose length is a 16-byte multiple starts 16-byte aligned).  A
// workgroup has NC waves; wave c owns chunk column c for every row it
// processes, and lane l owns block 64c + l, so the activation of that block
// is prepared once and kept in registers for the whole kernel.  Workgroups
// walk groups of G consecutive rows (persistent over the grid).
//
// Streaming.  Each wave copies its own chunks HBM -> LDS with
// global_load_lds_dwordx4 (cache policy nt, the weights are read once per
// call) into a private ring of NB buffers, keeping NB-1 chunks in flight, and
// waits for a chunk with its own vmcnt: no workgroup barrier inside the row
// loop.  The only barrier is per row group, for the cross-wave sum.
//
// Arithmetic.  Integer dot4 (v_dot4_i32_i8) on every block:
//   Q4_0: against the Q8_0 activation, exactly the reference's
//         vec_dot_q4_0_q8_0 (llama3pure-c-engine.c:1625-1643), block result
//         dw*dx*(float)isum;
//   Q8_0: against x as four int8 digits per 32-block,
//         x = 2^(e-6) (d0 + d1/2^7 + d2/2^14 + d3/2^21), exact to 2^-27 of the
//         block maximum; the four integer block dots are exact and combined
//         in fp32 (the reference dequantizes exactly and sums fp32 products,
//         c:2136-2176).
// Row totals: per-lane partials of the G rows are transposed-reduced across
// the wave, then summed over the NC waves in chunk order, so results do not
// depend on timing.
//
// Prologue (optional RMSNorm, c:3117-3129): every workgroup computes
// ss = sum(x^2) in one fixed order and r = 1/sqrt(ss/n + eps); lane l then
// forms w[j] * (r * x[j]) for its block and converts it.  The lane's x and
// norm loads are issued first, then the first weight copies, so HBM is busy
// while the activation is prepared.
#include "device_common.h"
#include "internal.h"

#include <map>
#include <mutex>
#include <tuple>

namespace {

using namespace l3pd;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kChunkBlocks = 64;
constexpr int kMaxOut = 4096;   // per-workgroup result slots kept in LDS

template <int QT>
struct Fmt;
// A chunk is copied with kX4 dwordx4 instructions (1024 B each) and one
// dword instruction (256 B) for the 128-byte tail; the tail instruction
// writes 128 B past the chunk, so buffers are kBufBytes long.
template <>
struct Fmt<L3P_Q8_0> {
    static constexpr int kBlockBytes = 34;
    static constexpr int kChunkBytes = 34 * kChunkBlocks;   // 2176 = 2*1024 + 128
    static constexpr int kX4 = 2;
    static constexpr int kBufBytes = kChunkBytes + 128;
};
template <>
struct Fmt<L3P_Q4_0> {
    static constexpr int kBlockBytes = 18;
    static constexpr int kChunkBytes = 18 * kChunkBlocks;   // 1152 = 1024 + 128
    static constexpr int kX4 = 1;
    static constexpr int kBufBytes = kChunkBytes + 128;
};

// Barrier for LDS traffic only (no wait on outstanding vector memory, which
// __syncthreads' release fence would add).
__device__ __forceinline__ void lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ void wait_lgkm() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until at most N of this wave's vector-memory operations are outstanding
// (s_waitcnt on gfx9: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// HBM -> LDS copy of one chunk (nbytes <= kChunkBytes, a 16-byte multiple)
// into this wave's buffer dst.  Always exactly kX4 + 1 instructions, every
// lane active: lanes past nbytes re-read the chunk's last bytes (the copy
// lands beyond nbytes in the buffer and is never read), so the number of
// outstanding copies per chunk is a constant the waits can count on.  Rows
// past the end of the matrix (a ragged last group) copy a valid dummy chunk.
template <int QT>
__device__ __forceinline__ void chunk_dma(uint32_t* dst, const uint8_t* __restrict__ src, int nbytes, int lane) {
#pragma unroll
    for (int j = 0; j < Fmt<QT>::kX4; ++j) {
        const int o = min(j * 1024 + lane * 16, nbytes - 16);
        __builtin_amdgcn_global_load_lds(src + o, (lds_void*)(dst + j * 256), 16, 0, 2);
    }
    const int o = min(Fmt<QT>::kX4 * 1024 + lane * 4, nbytes - 4);
    __builtin_amdgcn_global_load_lds(src + o, (lds_void*)(dst + Fmt<QT>::kX4 * 256), 4, 0, 2);
}

template <int N>
__device__ __forceinline__ constexpr int log2c() {
    return N >= 32 ? 5 : N >= 16 ? 4 : N >= 8 ? 3 : N >= 4 ? 2 : N >= 2 ? 1 : 0;
}
// Lane group of `lane` after xreduce<N>: which of the N values it holds.
template <int N>
__device__ __forceinline__ int rowof(int lane) {
    constexpr int L = log2c<N>();
    int r = 0;
#pragma unroll
    for (int s = 0; s < L; ++s) r |= ((lane >> (5 - s)) & 1) << (L - 1 - s);
    return r;
}
// Transpose-reduce N per-lane values over the wave: afterwards every lane of
// group g (64/N consecutive lanes) holds the wave total of value rowof<N>(lane).
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
                float lo = v[i], hi = v[i + half];
                // keep both as register values: a select between two array
                // elements would otherwise become a per-lane indexed load
                asm volatile("" : "+v"(lo), "+v"(hi));
                const float send = up ? lo : hi;
                const float keep = up ? hi : lo;
                v[i] = keep + __shfl_xor(send, m, 64);
            }
        }
    }
    float r = v[0];
#pragma unroll
    for (int m = 32 >> L; m > 0; m >>= 1) r += __shfl_xor(r, m, 64);
    return r;
}

struct Gemv4Args {
    const uint8_t* w[3];
    float* y[3];
    int rows[3];        // rows per segment; pair mode: rows[0] == rows[1]
    int nseg;
    int epilogue;       // GemvEpilogue
    int cols;
    int rows_total;     // sum of rows (pair: rows[0])
    int ngroups;
    const float* x;     // fp32 activation
    const float* norm;  // RMSNorm weights, or null for x as is
    float eps, inv_n;
};

// Row `i` of the concatenated row space -> (segment, local row).
__device__ __forceinline__ void seg_of(const Gemv4Args& a, int i, int& s, int& r) {
    s = 0;
    r = i;
    if (a.nseg > 1 && r >= a.rows[0]) {
        r -= a.rows[0];
        s = 1;
        if (a.nseg > 2 && r >= a.rows[1]) {
            r -= a.rows[1];
            s = 2;
        }
    }
}

// Row-chunk k of this workgroup's sequence: group j = blockIdx.x + (k / G) *
// gridDim.x, row slot i = k % G.  Pair mode: slots [0, G/2) are gate rows,
// [G/2, G) the matching up rows.  Sets src/nbytes to the chunk's bytes and
// returns true for a real row; past the end it returns false with src/nbytes
// pointing at the first chunk of the first matrix (a valid dummy copy).
template <int G, bool PAIR>
__device__ __forceinline__ bool chunk_src(const Gemv4Args& a, int k, int c, uint32_t rb, int chunk_bytes,
                                          const uint8_t*& src, int& nbytes) {
    const int j = blockIdx.x + (k / G) * gridDim.x;
    const int i = k % G;
    int s = 0, r = 0;
    bool ok = j < a.ngroups;
    if (ok) {
        if (PAIR) {
            s = i < G / 2 ? 0 : 1;
            r = j * (G / 2) + (i % (G / 2));
            ok = r < a.rows[0];
        } else {
            const int gi = j * G + i;
            ok = gi < a.rows_total;
            if (ok) seg_of(a, gi, s, r);
        }
    }
    if (!ok) {
        s = 0;
        r = 0;
        c = 0;
    }
    const uint32_t off = (uint32_t)c * (uint32_t)chunk_bytes;
    nbytes = (int)min((uint32_t)chunk_bytes, rb - off);
    src = a.w[s] + (size_t)r * rb + off;
    return ok;
}

// Activation of one 32-block in the form the weight type consumes.
struct XBlock {
    int q[4][8];   // Q8_0 weights: four digit planes; Q4_0 weights: q[0] = Q8_0 quants
    float s;       // Q8_0: digit scale; Q4_0: fp32 value of the Q8_0 scale
    int sum8;      // Q4_0: 8 * sum of quants
};

template <int QT>
__device__ __forceinline__ void prepare_block(const float* v, XBlock& xb) {
    if (QT == L3P_Q8_0) {
        int8_t dg[4][32];
        xb.s = digits32(v, dg);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                xb.q[k][e] = (int)((uint32_t)(uint8_t)dg[k][4 * e] | ((uint32_t)(uint8_t)dg[k][4 * e + 1] << 8) |
                                   ((uint32_t)(uint8_t)dg[k][4 * e + 2] << 16) |
                                   ((uint32_t)(uint8_t)dg[k][4 * e + 3] << 24));
        xb.sum8 = 0;
    } else {
        QBlock qb;
        quantize32(v, qb);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            xb.q[0][e] = (int)((uint32_t)(uint8_t)qb.q[4 * e] | ((uint32_t)(uint8_t)qb.q[4 * e + 1] << 8) |
                               ((uint32_t)(uint8_t)qb.q[4 * e + 2] << 16) |
                               ((uint32_t)(uint8_t)qb.q[4 * e + 3] << 24));
        xb.s = h2f_exact(qb.dh);
        xb.sum8 = 8 * qb.sum;
    }
}

// Dot of the block at LDS byte offset `boff` (2-byte aligned) with the lane's
// activation block.
template <int QT>
__device__ __forceinline__ float block_dot(const uint32_t* lds, uint32_t boff, const XBlock& xb) {
    const uint32_t E = boff >> 2;
    const bool odd = (boff & 2u) != 0;   // block starts 2 bytes into a dword
    if (QT == L3P_Q8_0) {
        uint32_t dw[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) dw[k] = lds[E + k];
        const float d = h2f(odd ? (dw[0] >> 16) : dw[0]);
        int I[4] = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int q = (int)(odd ? dw[k + 1] : __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2));
#pragma unroll
            for (int g = 0; g < 4; ++g) I[g] = __builtin_amdgcn_sdot4(q, xb.q[g][k], I[g], false);
        }
        const float c7 = 0.0078125f;
        const float f = (float)I[0] + ((float)I[1] + ((float)I[2] + (float)I[3] * c7) * c7) * c7;
        return f * (d * xb.s);
    } else {
        uint32_t dw[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) dw[k] = lds[E + k];
        const float dwt = h2f(odd ? (dw[0] >> 16) : dw[0]);
        int isum = -xb.sum8;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = odd ? dw[k + 1] : __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2);
            isum = __builtin_amdgcn_sdot4((int)(q & 0x0f0f0f0fu), xb.q[0][k], isum, false);
            isum = __builtin_amdgcn_sdot4((int)((q >> 4) & 0x0f0f0f0fu), xb.q[0][4 + k], isum, false);
        }
        return dwt * xb.s * (float)isum;
    }
}

template <int QT, int G, int NB, bool PAIR>
__global__ void __launch_bounds__(1024) gemv4_kernel(Gemv4Args a) {
    constexpr int CB = Fmt<QT>::kChunkBytes;
    constexpr int BB = Fmt<QT>::kBlockBytes;
    constexpr int CDW = Fmt<QT>::kBufBytes / 4;
    constexpr int CI = Fmt<QT>::kX4 + 1;   // copy instructions per chunk
    constexpr int NOUT = PAIR ? G / 2 : G;
    extern __shared__ __align__(16) uint32_t lds[];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, nw = blockDim.x >> 6;
    const int nb = a.cols >> 5;
    const uint32_t rb = (uint32_t)nb * BB;
    uint32_t* ring = lds + (size_t)w * NB * CDW;                          // this wave's chunk buffers
    float* red = reinterpret_cast<float*>(lds + (size_t)nw * NB * CDW);   // [2][nw][G]
    float* ssred = red + 2 * nw * G;                                      // [nw]
    float* out_lds = ssred + nw;                                          // [groups of this WG][NOUT]

    // ---- this lane's activation block (and the norm weights), issued first:
    // they come from L2 while the weight copies below are in flight
    const int blk = w * kChunkBlocks + lane;
    const bool active = blk < nb;
    float v[32];
    float4 nv[8];
    if (active) {
        const float4* xp = reinterpret_cast<const float4*>(a.x + 32 * blk);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float4 q = xp[e];
            v[4 * e] = q.x; v[4 * e + 1] = q.y; v[4 * e + 2] = q.z; v[4 * e + 3] = q.w;
        }
        if (a.norm) {
            const float4* np = reinterpret_cast<const float4*>(a.norm + 32 * blk);
#pragma unroll
            for (int e = 0; e < 8; ++e) nv[e] = np[e];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = 0.0f;
    }
    // ---- weight copies: the first NB-1 chunks of this workgroup's sequence,
    // CI instructions each.  nk = number of row-chunks this wave processes.
    const int ngroups_mine =
        a.ngroups > (int)blockIdx.x ? (a.ngroups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
    const int nk = ngroups_mine * G;
#pragma unroll
    for (int b = 0; b < NB - 1; ++b) {
        if (b < nk) {
            const uint8_t* src;
            int nbytes;
            chunk_src<G, PAIR>(a, b, w, rb, CB, src, nbytes);
            chunk_dma<QT>(ring + b * CDW, src, nbytes, lane);
        }
    }

    // ---- optional RMSNorm.  Every block of x belongs to exactly one lane, so
    // ss = sum over lanes of the lane's 32 squares, then over lanes and waves
    // in a fixed order: the same value in every workgroup.
    if (a.norm) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) ss += v[j] * v[j];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) ssred[w] = ss;
        lds_sync();
        ss = 0.0f;
        for (int i = 0; i < nw; ++i) ss += ssred[i];
        const float r = 1.0f / sqrtf(ss * a.inv_n + a.eps);
        if (active) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[4 * e] = nv[e].x * (r * v[4 * e]);
                v[4 * e + 1] = nv[e].y * (r * v[4 * e + 1]);
                v[4 * e + 2] = nv[e].z * (r * v[4 * e + 2]);
                v[4 * e + 3] = nv[e].w * (r * v[4 * e + 3]);
            }
        }
    }
    XBlock xb;
    prepare_block<QT>(v, xb);

    // ---- row loop: G rows per group, chunk k = gl*G + i of this WG's sequence
    for (int gl = 0; gl < ngroups_mine; ++gl) {
        float acc[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int k = gl * G + i;
            // chunk k is in LDS once only the younger chunks' copies remain:
            // NB-2 of them in steady state, none near the end of the sequence
            if (k + NB - 2 < nk) wait_vm<(NB - 2) * CI>();
            else wait_vm<0>();
            const uint8_t* src;
            int nbytes;
            const bool real = chunk_src<G, PAIR>(a, k, w, rb, CB, src, nbytes);
            float d = 0.0f;
            if (real && active) d = block_dot<QT>(ring + (k % NB) * CDW, (uint32_t)lane * BB, xb);
            wait_lgkm();   // this chunk's LDS reads are done before its buffer is refilled
            const int kn = k + NB - 1;
            if (kn < nk) {
                chunk_src<G, PAIR>(a, kn, w, rb, CB, src, nbytes);
                chunk_dma<QT>(ring + (kn % NB) * CDW, src, nbytes, lane);
            }
            acc[i] = d;
        }
        // group done: wave totals -> LDS -> sum over the chunk waves in order
        float* rd = red + (gl & 1) * nw * G;
        const float tot = xreduce<G>(acc, lane);
        if ((lane & ((64 / G) - 1)) == 0) rd[w * G + rowof<G>(lane)] = tot;
        lds_sync();
        if (t < NOUT) {
            float s0 = 0.0f;
            for (int c = 0; c < nw; ++c) s0 += rd[c * G + t];
            float res = s0;
            if (PAIR) {
                float s1 = 0.0f;
                for (int c = 0; c < nw; ++c) s1 += rd[c * G + G / 2 + t];
                res = a.epilogue == EPI_GEGLU ? ref_geglu(s0, s1) : ref_swiglu(s0, s1);
            }
            out_lds[gl * NOUT + t] = res;
        }
    }
    // ---- results of this workgroup's groups (every copy has been waited for)
    lds_sync();
    for (int j = t; j < ngroups_mine * NOUT; j += blockDim.x) {
        const int gk = j / NOUT, i = j % NOUT;
        const int grp = blockIdx.x + gk * gridDim.x;
        if (PAIR) {
            const int row = grp * NOUT + i;
            if (row < a.rows[0]) a.y[0][row] = out_lds[j];
        } else {
            const int gi = grp * G + i;
            if (gi >= a.rows_total) continue;
            int s, row;
            seg_of(a, gi, s, row);
            float* y = a.y[s] + row;
            if (a.epilogue == EPI_ADD) *y += out_lds[j];
            else *y = out_lds[j];
        }
    }
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------
int cus() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 0;
        if (n <= 0) n = 256;
    }
    return n;
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

int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

template <int QT, int G, int NB, bool PAIR>
void launch4(Gemv4Args a, hipStream_t st) {
    constexpr int NOUT = PAIR ? G / 2 : G;
    const int nb = a.cols / 32;
    const int nw = (nb + kChunkBlocks - 1) / kChunkBlocks;
    const int threads = nw * 64;
    const size_t base = (size_t)nw * NB * Fmt<QT>::kBufBytes + (size_t)2 * nw * G * 4 + (size_t)nw * 4;
    auto lds_for = [&](int grid) { return base + (size_t)((a.ngroups + grid - 1) / grid) * NOUT * 4; };
    auto kern = gemv4_kernel<QT, G, NB, PAIR>;
    const int per_cu = occupancy(kern, threads, lds_for(cus()));
    int grid = std::min(a.ngroups, per_cu * cus());
    grid = std::max(grid, (a.ngroups * NOUT + kMaxOut - 1) / kMaxOut);
    const size_t lds = lds_for(grid);
    if (lds > 65536)
        L3P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(threads), lds, st, a);
    L3P_HIP(hipGetLastError());
}

template <int QT, int G, bool PAIR>
void launch4_nb(Gemv4Args a, int nbuf, hipStream_t st) {
    switch (nbuf) {
    case 3: launch4<QT, G, 3, PAIR>(a, st); break;
    case 6: launch4<QT, G, 6, PAIR>(a, st); break;
    default: launch4<QT, G, 4, PAIR>(a, st); break;
    }
}

template <int QT>
void launch4_type(Gemv4Args a, bool pair, int G, int nbuf, hipStream_t st) {
    const int units = pair ? a.rows[0] : a.rows_total;
    const int per = pair ? G / 2 : G;
    a.ngroups = (units + per - 1) / per;
    if (pair) {   // G counts gate and up rows together: 2 or 4 output rows per group
        switch (G) {
        case 4: launch4_nb<QT, 4, true>(a, nbuf, st); break;
        default: launch4_nb<QT, 8, true>(a, nbuf, st); break;
        }
    } else {
        switch (G) {
        case 4: launch4_nb<QT, 4, false>(a, nbuf, st); break;
        case 16: launch4_nb<QT, 16, false>(a, nbuf, st); break;
        default: launch4_nb<QT, 8, false>(a, nbuf, st); break;
        }
    }
}

}  // namespace

bool gemv4_supported(int type, int cols) {
    if (type != L3P_Q8_0 && type != L3P_Q4_0) return false;
    return cols > 0 && cols % 256 == 0 && cols <= 64 * 1024;
}

void launch_gemv4(int type, const GemvBatch& b, int cols, const float* x, const float* norm, float eps,
                  hipStream_t st) {
    Gemv4Args a{};
    for (int s = 0; s < b.nseg; ++s) {
        a.w[s] = b.seg[s].w;
        a.y[s] = b.seg[s].y;
        a.rows[s] = b.seg[s].rows;
        L3P_REQUIRE(((uintptr_t)a.w[s] & 15) == 0, L3P_E_INVALID, "gemv: weights must be 16-byte aligned");
    }
    a.nseg = b.nseg;
    a.epilogue = b.epilogue;
    a.cols = cols;
    a.rows_total = 0;
    if (b.pair) a.rows_total = b.seg[0].rows;
    else
        for (int s = 0; s < b.nseg; ++s) a.rows_total += b.seg[s].rows;
    if (a.rows_total == 0) return;
    a.x = x;
    a.norm = norm;
    a.eps = eps;
    a.inv_n = 1.0f / (float)cols;
    // rows per group: enough groups to give every CU work, then the largest
    const int units = a.rows_total;
    int G = env_int("L3P_GEMV4_G", 0);
    if (G != 4 && G != 8 && G != 16) G = units >= 16 * 4 * cus() ? 16 : units >= 8 * 2 * cus() ? 8 : 4;
    const int nbuf = env_int("L3P_GEMV4_NB", 4);
    if (type == L3P_Q8_0) launch4_type<L3P_Q8_0>(a, b.pair != 0, G, nbuf, st);
    else launch4_type<L3P_Q4_0>(a, b.pair != 0, G, nbuf, st);
}
