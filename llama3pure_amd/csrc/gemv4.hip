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
// Arithmetic per block:
//   Q4_0: integer dot4 (v_dot4_i32_i8) against the Q8_0 activation, exactly
//         the reference's vec_dot_q4_0_q8_0 (llama3pure-c-engine.c:1625-1643),
//         block result dw*dx*(float)isum;
//   Q8_0: d * sum_j q_j x_j with fp32 FMAs on the fp32 activation (the
//         reference dequantizes exactly and sums fp32 products, c:2136-2176).
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

// Byte offsets this lane copies within a chunk of nbytes (<= kChunkBytes, a
// 16-byte multiple; the same for every row a wave copies): kX4 dwordx4
// pieces and one dword piece, clamped so lanes past nbytes re-read the
// chunk's last bytes (that copy lands past nbytes in the buffer and is never
// read).  Every chunk is therefore exactly kX4 + 1 instructions with all
// lanes active, a constant the waits count on.
struct DmaLane {
    int o0, o1;   // the dwordx4 pieces (o1 unused for Q4_0's single one)
    int ot;       // the dword piece
};
template <int QT>
__device__ __forceinline__ DmaLane dma_lane(int lane, int nbytes) {
    DmaLane d;
    d.o0 = min(lane * 16, nbytes - 16);
    d.o1 = min(1024 + lane * 16, nbytes - 16);
    d.ot = min(Fmt<QT>::kX4 * 1024 + lane * 4, nbytes - 4);
    return d;
}
// HBM -> LDS copy of one chunk into this wave's buffer dst (lane i of an
// instruction writes the instruction's LDS base + 16 i, or + 4 i for the dword piece).
template <int QT>
__device__ __forceinline__ void chunk_dma(uint32_t* dst, const uint8_t* src, DmaLane d) {
    __builtin_amdgcn_global_load_lds(src + d.o0, (lds_void*)dst, 16, 0, 2);
    if (Fmt<QT>::kX4 > 1) __builtin_amdgcn_global_load_lds(src + d.o1, (lds_void*)(dst + 256), 16, 0, 2);
    __builtin_amdgcn_global_load_lds(src + d.ot, (lds_void*)(dst + Fmt<QT>::kX4 * 256), 4, 0, 2);
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

// The rows a wave streams, as wave-uniform values.
struct Cursor {
    const uint8_t *w0, *w1, *w2;
    int rows0, rows1, rows_total, ngroups, bid, gdim;
    uint32_t rb;      // row bytes
    uint32_t coff;    // byte offset of this wave's chunk column in a row
};

// Row-chunk k of this workgroup's sequence: group j = blockIdx.x + (k / G) *
// gridDim.x, row slot i = k % G.  Pair mode: slots [0, G/2) are gate rows,
// [G/2, G) the matching up rows.  Sets src to the chunk and returns true for
// a real row; past the end it returns false with src at the same chunk column
// of the first row (a valid dummy copy of the same size).
template <int G, bool PAIR>
__device__ __forceinline__ bool chunk_src(const Cursor& cc, int k, const uint8_t*& src) {
    const int j = cc.bid + (k / G) * cc.gdim;
    const int i = k % G;
    const uint8_t* base = cc.w0;
    int r;
    bool ok = j < cc.ngroups;
    if (PAIR) {
        r = j * (G / 2) + (i % (G / 2));
        if (i >= G / 2) base = cc.w1;
        ok = ok && r < cc.rows0;
    } else {
        r = j * G + i;
        ok = ok && r < cc.rows_total;
        if (r >= cc.rows0) {
            r -= cc.rows0;
            base = cc.w1;
            if (r >= cc.rows1) {
                r -= cc.rows1;
                base = cc.w2;
            }
        }
    }
    if (!ok) {
        base = cc.w0;
        r = 0;
    }
    src = base + (size_t)r * cc.rb + cc.coff;
    return ok;
}

// Activation of one 32-block in the form the weight type consumes.
struct XBlock {
    float x[32];   // Q8_0 weights: the fp32 values
    int q[8];      // Q4_0 weights: the Q8_0 quants, four per dword
    float s;       // Q4_0: fp32 value of the Q8_0 scale
    int sum8;      // Q4_0: 8 * sum of quants
};

template <int QT>
__device__ __forceinline__ void prepare_block(const float* v, XBlock& xb) {
    if (QT == L3P_Q8_0) {
#pragma unroll
        for (int j = 0; j < 32; ++j) xb.x[j] = v[j];
    } else {
        QBlock qb;
        quantize32(v, qb);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            xb.q[e] = (int)((uint32_t)(uint8_t)qb.q[4 * e] | ((uint32_t)(uint8_t)qb.q[4 * e + 1] << 8) |
                            ((uint32_t)(uint8_t)qb.q[4 * e + 2] << 16) | ((uint32_t)(uint8_t)qb.q[4 * e + 3] << 24));
        xb.s = h2f_exact(qb.dh);
        xb.sum8 = 8 * qb.sum;
    }
}

// Where lane l's block sits in a chunk buffer: its fp16 scale is the
// halfword at byte BB*l; its quants start at byte BB*l + 2, which is
// dword-aligned for odd l and 2 bytes into a dword for even l.  Reading nine
// dwords from `first` and taking alignbyte(dw[k+1], dw[k], shift) gives the
// k-th quant dword for both parities with one instruction and no branch.
struct LaneBlock {
    uint32_t half;    // halfword index of the scale
    uint32_t first;   // dword index of the first dword read
    uint32_t shift;   // byte shift for v_alignbyte: 2 (even l) or 0 (odd l)
};
template <int QT>
__device__ __forceinline__ LaneBlock lane_block(int lane) {
    const uint32_t b = (uint32_t)lane * Fmt<QT>::kBlockBytes;
    const bool odd = (b & 2u) != 0;
    return LaneBlock{b >> 1, (b >> 2) + (odd ? 1u : 0u), odd ? 0u : 2u};
}

// Dot of the lane's block in the chunk buffer `buf` with the lane's activation:
//   Q8_0: d * sum_j q_j x_j with fp32 FMAs (the reference dequantizes exactly,
//         q*d, and sums fp32 products, c:2136-2176; fp32 summation order is
//         the only difference);
//   Q4_0: the reference's integer block dot against the Q8_0 activation,
//         dw*dx*(float)isum (vec_dot_q4_0_q8_0, c:1625-1643).
template <int QT>
__device__ __forceinline__ float block_dot(const uint32_t* buf, const LaneBlock& lb, const XBlock& xb) {
    const float d = h2f(reinterpret_cast<const uint16_t*>(buf)[lb.half]);
    const uint32_t* p = buf + lb.first;
    if (QT == L3P_Q8_0) {
        uint32_t dw[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) dw[k] = p[k];
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t q = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], lb.shift);
            s0 = fmaf((float)(int8_t)(q & 0xffu), xb.x[4 * k], s0);
            s1 = fmaf((float)(int8_t)((q >> 8) & 0xffu), xb.x[4 * k + 1], s1);
            s2 = fmaf((float)(int8_t)((q >> 16) & 0xffu), xb.x[4 * k + 2], s2);
            s3 = fmaf((float)(int8_t)(q >> 24), xb.x[4 * k + 3], s3);
        }
        return ((s0 + s1) + (s2 + s3)) * d;
    } else {
        uint32_t dw[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) dw[k] = p[k];
        int isum = -xb.sum8;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], lb.shift);
            isum = __builtin_amdgcn_sdot4((int)(q & 0x0f0f0f0fu), xb.q[k], isum, false);
            isum = __builtin_amdgcn_sdot4((int)((q >> 4) & 0x0f0f0f0fu), xb.q[4 + k], isum, false);
        }
        return d * xb.s * (float)isum;
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
    const int t = threadIdx.x, lane = t & 63, nw = blockDim.x >> 6;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nb = a.cols >> 5;
    const uint32_t rb = (uint32_t)nb * BB;
    uint32_t* ring = lds + (size_t)w * NB * CDW;                          // this wave's chunk buffers
    Cursor cc;
    cc.w0 = a.w[0];
    cc.w1 = a.w[1];
    cc.w2 = a.w[2];
    cc.rows0 = a.rows[0];
    cc.rows1 = a.rows[1];
    cc.rows_total = a.rows_total;
    cc.ngroups = a.ngroups;
    cc.bid = blockIdx.x;
    cc.gdim = gridDim.x;
    cc.rb = rb;
    cc.coff = (uint32_t)w * (uint32_t)CB;
    const DmaLane dl = dma_lane<QT>(lane, (int)min((uint32_t)CB, rb - cc.coff));
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
            chunk_src<G, PAIR>(cc, b, src);
            chunk_dma<QT>(ring + b * CDW, src, dl);
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
    const LaneBlock lb = lane_block<QT>(lane);

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
            const bool real = chunk_src<G, PAIR>(cc, k, src);
            // every lane reads inside the buffer, so the dot runs unconditionally
            // and lanes past the row or rows past the matrix drop their value
            float dv = block_dot<QT>(ring + (k % NB) * CDW, lb, xb);
            // pin the dot here: left alone, the compiler sinks every dot of the
            // group to its end and keeps all their quants live in registers
            asm volatile("" : "+v"(dv));
            const float d = (real && active) ? dv : 0.0f;
            wait_lgkm();   // this chunk's LDS reads are done before its buffer is refilled
            const int kn = k + NB - 1;
            if (kn < nk) {
                chunk_src<G, PAIR>(cc, kn, src);
                chunk_dma<QT>(ring + (kn % NB) * CDW, src, dl);
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
    case 8: launch4<QT, G, 8, PAIR>(a, st); break;
    default: launch4<QT, G, 4, PAIR>(a, st); break;
    }
}

template <int QT>
void launch4_type(Gemv4Args a, bool pair, int G, int nbuf, hipStream_t st) {
    const int units = pair ? a.rows[0] : a.rows_total;
    const int per = pair ? G / 2 : G;
    a.ngroups = (units + per - 1) / per;
    // the deepest ring (3, 4, 6, 8 or 12 buffers per wave) not above nbuf
    // whose buffers fit the 160 KB of LDS with room for the result slots
    const int nw = (a.cols / 32 + kChunkBlocks - 1) / kChunkBlocks;
    static const int depths[] = {8, 6, 4, 3};
    int nb = 3;
    for (int d : depths)
        if (d <= nbuf && (size_t)nw * d * Fmt<QT>::kBufBytes + 16384 <= 160 * 1024) {
            nb = d;
            break;
        }
    nbuf = nb;
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
    // Rows per group G: the largest of 16, 8, 4 that still gives about six
    // waves per CU (groups x column chunks); ring depth 3 at G = 4, else 4.
    // (Measured on MI355X at the Llama-3-8B shapes.)
    const int nw = (cols / 32 + kChunkBlocks - 1) / kChunkBlocks;
    const int units = a.rows_total;
    const int per_g = b.pair ? 2 : 1;   // pair groups hold G/2 rows of each matrix
    auto waves = [&](int g) { return (long)(units * per_g + g - 1) / g * nw; };
    int G = env_int("L3P_GEMV4_G", 0);
    if (G != 4 && G != 8 && G != 16) {
        G = 4;
        for (int g : {16, 8})
            if ((!b.pair || g <= 8) && waves(g) >= 6L * cus()) {
                G = g;
                break;
            }
    }
    const int nbuf = env_int("L3P_GEMV4_NB", G == 4 ? 3 : 4);
    if (type == L3P_Q8_0) launch4_type<L3P_Q8_0>(a, b.pair != 0, G, nbuf, st);
    else launch4_type<L3P_Q4_0>(a, b.pair != 0, G, nbuf, st);
}
