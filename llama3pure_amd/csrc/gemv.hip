// gemv.hip — streaming decode GEMVs over GGUF Q8_0, Q4_0, Q4_K and Q6_K rows
// (gfx950), split over 2048-element column chunks, with the activation's
// RMSNorm (and, for Q4_0, its Q8_0 form) computed in the prologue.
//
// Work split.  A row of `cols` elements is cut into NC = ceil(cols/2048)
// chunks of 2048 elements: 64 Q8_0 / Q4_0 blocks (2176 / 1152 B) or 8 Q4_K /
// Q6_K super-blocks (1152 / 1680 B).  A workgroup has NC waves; wave c owns
// chunk column c of every row it processes, and lane l owns the 32 elements
// [2048c + 32l, +32) (a Q8_0/Q4_0 block, a Q4_K sub-block, a quarter of a
// Q6_K half super-block), so the activation of those elements is prepared
// once and kept in registers for the whole kernel.  Workgroups walk groups of
// G consecutive rows (persistent over the grid).
//
// Streaming.  Each wave copies its own chunks HBM -> LDS with
// global_load_lds (dwordx4 pieces and a dword piece, cache policy nt: the
// weights are read once per call) into a private ring of NB buffers.  Before
// computing chunk k it refills the buffer of chunk k-1 with chunk k+NB-1, so
// NB-1 chunks are in flight during the compute, and waits for chunk k with
// its own vmcnt: no workgroup barrier inside the row loop.  The only barrier is per row group,
// for the cross-wave sum.
//
// Row alignment.  When a row's length in bytes is a multiple of 16 (cols a
// multiple of 256 for Q8_0/Q4_0, of 2048 for Q6_K, always for Q4_K) every
// chunk starts 16-byte aligned.  Otherwise (UA kernels) a chunk is copied from
// its address rounded down to 16, its data lands `sh` = address % 16 bytes
// into the buffer, and each lane recomputes where its elements sit.  Copies
// then reach at most to the end of the 16-byte granule that holds the row's
// last byte, which lies in the same page as that byte.
//
// Arithmetic per lane (32 elements j):
//   Q8_0: d * sum q_j x_j, fp32 FMAs on the fp32 activation (the reference
//         dequantizes exactly, q*d, and sums fp32 products, c:2136-2176);
//   Q4_0: the reference's integer block dot against the Q8_0 activation,
//         dw*dx*(float)isum (vec_dot_q4_0_q8_0, c:1625-1643);
//   Q4_K: (d*sc) * sum q_j x_j - (dmin*m) * sum x_j with the sub-block's
//         6-bit scale and min (get_scale_min_k4 + dequantize_row_q4_K,
//         c:705-746);
//   Q6_K: d * sum over the two 16-element halves of sc_h * (sum u_j x_j -
//         32 sum x_j), u = q + 32 the 6-bit code (dequantize_row_q6_K,
//         c:873-904).
// The reference rounds w_j = dequant(q_j) and then sums w_j x_j in fp32; the
// factored forms differ from it only in fp32 rounding order.
// Row totals: per-lane partials of the G rows are transposed-reduced across
// the wave, then summed over the NC waves in chunk order, so results do not
// depend on timing.
//
// Prologue (optional RMSNorm, c:3117-3129): every workgroup computes
// ss = sum(x^2) in one fixed order and r = 1/sqrt(ss/n + eps).  Q4_0 lanes
// form w[j] * (r * x[j]) and quantize it as the reference does; the fp32
// types use w[j] * x[j] and multiply each row total by r (the product is
// linear in x), so no wave waits for the others before its first chunk.
// The lane's x and norm loads are issued first, then the first weight
// copies, and the prologue waits only for the loads, so the copies stay in
// flight while the activation is prepared.
//
// Normed residual hand-over (fp32-activation types): a residual-add GEMV
// (EPI_ADD) may also write x' * w_next for its outputs x' and its
// workgroup's sum of x'^2 in a fixed order; the next GEMV then loads that
// vector and those sums (256 per load) instead of x and its norm weights,
// and scales its row totals by r from the sums.
#include "device_common.h"
#include "internal.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

namespace {

using namespace l3pd;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kChunkElems = 2048;   // 64 lanes x 32 elements
constexpr int kMaxWaves = 16;       // chunk columns per row: cols <= 32768
constexpr int kMaxOut = 4096;       // per-workgroup result slots kept in LDS

// Storage unit of a type (a block or super-block) and how a chunk is copied:
// kX4 dwordx4 instructions (1024 B each) and, with kTail, one dword
// instruction (256 B).  The pieces cover kChunkBytes + 14 (the largest start
// offset of an unaligned chunk); clamped lanes write past the data, so a
// buffer is kBufBytes long.
// ALIGNED: the type's rows are always 16-byte multiples (no UA kernel).
template <int UE, int UB, int X4, int TAIL, bool ALIGNED = false>
struct FmtBase {
    static constexpr int kUnitElems = UE;
    static constexpr int kUnitBytes = UB;
    static constexpr int kChunkBytes = kChunkElems / UE * UB;
    static constexpr int kX4 = X4;
    static constexpr int kTail = TAIL;
    static constexpr int kCI = X4 + TAIL;   // copy instructions per chunk
    static constexpr int kBufBytes = X4 * 1024 + TAIL * 256;
    static constexpr bool kAligned = ALIGNED;
    static_assert(kChunkBytes + (ALIGNED ? 0 : 14) <= kBufBytes, "copy pieces must cover an unaligned chunk");
};
template <int QT>
struct Fmt;
template <> struct Fmt<L3P_Q8_0> : FmtBase<32, 34, 2, 1> {};            // 2176 B chunks
template <> struct Fmt<L3P_Q4_0> : FmtBase<32, 18, 1, 1> {};            // 1152 B
template <> struct Fmt<L3P_Q4_1> : FmtBase<32, 20, 2, 0> {};            // 1280 B
template <> struct Fmt<L3P_Q5_0> : FmtBase<32, 22, 2, 0> {};            // 1408 B
template <> struct Fmt<L3P_Q5_1> : FmtBase<32, 24, 2, 0> {};            // 1536 B
template <> struct Fmt<L3P_IQ4_NL> : FmtBase<32, 18, 1, 1> {};          // 1152 B
template <> struct Fmt<L3P_Q2_K> : FmtBase<256, 84, 1, 0> {};           // 672 B
template <> struct Fmt<L3P_Q3_K> : FmtBase<256, 110, 1, 0> {};          // 880 B
template <> struct Fmt<L3P_Q4_K> : FmtBase<256, 144, 1, 1, true> {};    // 1152 B
template <> struct Fmt<L3P_Q5_K> : FmtBase<256, 176, 2, 0, true> {};    // 1408 B
template <> struct Fmt<L3P_Q6_K> : FmtBase<256, 210, 2, 0> {};          // 1680 B
template <> struct Fmt<L3P_F16> : FmtBase<32, 64, 4, 0, true> {};       // 4096 B
template <> struct Fmt<L3P_BF16> : FmtBase<32, 64, 4, 0, true> {};      // 4096 B
template <> struct Fmt<L3P_F32> : FmtBase<32, 128, 8, 0, true> {};      // 8192 B

// Types whose reference dot takes the activation as Q8_0 (vec_dot_*_q8_0:
// q8_func without a row dequantizer, c:2091-2133); the others dot fp32.
template <int QT>
__host__ __device__ constexpr bool q8_act() {
    return QT == L3P_Q4_0 || QT == L3P_Q4_1 || QT == L3P_Q5_0 || QT == L3P_Q5_1 || QT == L3P_IQ4_NL;
}

template <int QT>
__host__ __device__ __forceinline__ uint32_t row_bytes(int cols) {
    return (uint32_t)(cols / Fmt<QT>::kUnitElems) * Fmt<QT>::kUnitBytes;
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

// Wait for the copy of a chunk when `younger` copies (CI instructions each)
// were issued after it: vmcnt(min(younger, J) * CI), as a chain of scalar
// compares that ends at the first hit (the common case is younger >= J).
template <int J, int CI>
__device__ __forceinline__ void wait_chunk(int younger) {
    if constexpr (J == 0) {
        wait_vm<0>();
    } else {
        if (younger >= J) wait_vm<J * CI>();
        else wait_chunk<J - 1, CI>(younger);
    }
}

// Prologue loads the compiler does not track.  Issued before the weight
// copies and consumed after them, an ordinary load would be waited for with
// vmcnt(0), since the compiler's wait counting leaves the LDS-DMA copies out,
// and that also waits for every copy issued after it.  These loads are
// waited for by wait_prologue, which leaves the copies in flight; pin8 then
// orders each use after that wait.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void load8_async(f32x4 (&q)[8], const float* p) {
#pragma unroll
    for (int e = 0; e < 8; ++e) asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(q[e]) : "v"(p), "i"(16 * e));
}
// vmcnt(min(younger, J) * CI): every load older than the last `younger`
// chunk copies (CI instructions each) has landed
template <int J, int CI>
__device__ __forceinline__ void wait_prologue(int younger) {
    if constexpr (J == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        if (younger >= J) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(J * CI) : "memory");
        else wait_prologue<J - 1, CI>(younger);
    }
}
__device__ __forceinline__ void pin8(f32x4 (&q)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(q[e]));
}

// Byte offsets this lane copies, from the copy base, for a chunk whose data
// is bytes [0, span) of the copy: dwordx4 pieces over [0, 1024 kX4), the
// dword piece over [1024 kX4, +256).  Offsets are clamped to the last whole
// piece that ends within span rounded up to 16 (or 4), so lanes past the data
// re-read its last bytes (landing past span in the buffer, never read).
// Every chunk is therefore exactly kCI instructions with all lanes active, a
// constant the waits count on.
struct DmaLane {
    int o[8];   // the dwordx4 pieces (kX4 <= 8 of them)
    int ot;     // the dword piece (unused without a tail)
};
template <int QT>
__device__ __forceinline__ DmaLane dma_lane(int lane, int span) {
    static_assert(Fmt<QT>::kX4 <= 8, "at most eight dwordx4 pieces");
    const int e16 = ((span + 15) & ~15) - 16, e4 = ((span + 3) & ~3) - 4;
    DmaLane d;
#pragma unroll
    for (int i = 0; i < Fmt<QT>::kX4; ++i) d.o[i] = min(1024 * i + lane * 16, e16);
    d.ot = min(Fmt<QT>::kX4 * 1024 + lane * 4, e4);
    return d;
}
// HBM -> LDS copy of one chunk into this wave's buffer dst (lane i of an
// instruction writes the instruction's LDS base + 16 i, or + 4 i for the dword piece).
template <int QT>
__device__ __forceinline__ void chunk_dma(uint32_t* dst, const uint8_t* src, DmaLane d) {
#pragma unroll
    for (int i = 0; i < Fmt<QT>::kX4; ++i)
        __builtin_amdgcn_global_load_lds(src + d.o[i], (lds_void*)(dst + 256 * i), 16, 0, 2);
    if (Fmt<QT>::kTail)
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
                v[i] = keep + lane_partner_m(send, m);
            }
        }
    }
    float r = v[0];
#pragma unroll
    for (int m = 32 >> L; m > 0; m >>= 1) r += lane_partner_m(r, m);
    return r;
}

struct GemvArgs {
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
    // x := x + post_w * (r_y * post_y) first, r_y = 1/sqrt(sum(post_y^2)/cols
    // + eps), written to post_out by workgroup 0 (post_y null: x as is)
    const float *post_y, *post_w;
    float* post_out;
    // residual-add producers: also xw[i] = y[i] * xw_w[i], ssp[blockIdx.x] =
    // the workgroup's sum of y[i]^2 (xw null: neither)
    float* xw;
    const float* xw_w;
    float* ssp;
    // consumers: x is the residual times the norm weights and the RMSNorm's
    // sum of squares is the sum of ss[0..n_ss), read 256 per load over
    // ss_loads loads (ss null: no such norm).  Entries past n_ss are never
    // counted: they may hold an earlier producer's sums from a larger grid.
    const float* ss;
    int ss_loads;
    int n_ss;
    // > 0 (not pair mode): workgroup b takes the rows [b * rpw, (b + 1) *
    // rpw) in groups of G, the last group cut short; 0: the groups b, b +
    // gridDim.x, b + 2 * gridDim.x, ... of G consecutive rows each
    int rpw;
};

// Row `i` of the concatenated row space -> (segment, local row).
__device__ __forceinline__ void seg_of(const GemvArgs& a, int i, int& s, int& r) {
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
    int rbeg, nmine;  // row ranges (rpw > 0): first row and rows of this workgroup, else nmine = -1
    uint32_t rb;      // row bytes
    uint32_t coff;    // byte offset of this wave's chunk column in a row
};

// Row-chunk k of this workgroup's sequence: group j = blockIdx.x + (k / G) *
// gridDim.x, row slot i = k % G.  Pair mode: slots [0, G/2) are gate rows,
// [G/2, G) the matching up rows.  Sets src to the chunk and returns true for
// a real row; past the end it returns false with src at the same chunk column
// of the first row (a valid dummy copy of the same size).  RG: the kernel
// supports row ranges (see gemv_kernel).
template <int G, bool PAIR, bool RG = false>
__device__ __forceinline__ bool chunk_src(const Cursor& cc, int k, const uint8_t*& src) {
    const int j = cc.bid + (k / G) * cc.gdim;
    const int i = k % G;
    const uint8_t* base = cc.w0;
    int r;
    bool ok = j < cc.ngroups;
    if (RG && !PAIR && cc.nmine >= 0) {   // row ranges: chunk k is row rbeg + k
        r = cc.rbeg + k;
        ok = k < cc.nmine;
        if (ok && r >= cc.rows0) {
            r -= cc.rows0;
            base = cc.w1;
            if (r >= cc.rows1) {
                r -= cc.rows1;
                base = cc.w2;
            }
        }
    } else if (PAIR) {
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

// Activation of one lane's 32 elements in the form the weight type consumes.
struct XBlock {
    float x[32];    // fp32-activation types: the values
    int q[8];       // Q8_0-activation types: the Q8_0 quants, four per dword
    float s;        //   fp32 value of the Q8_0 scale
    int sum8;       //   8 * sum of quants
    float xs;       // sum of the 32 values (Q4_K, Q5_K)
    float xs0, xs1; // sums of values 0..15 and 16..31 (Q6_K)
};

template <int QT>
__device__ __forceinline__ void prepare_block(const float* v, XBlock& xb) {
    if (q8_act<QT>()) {
        QBlock qb;
        quantize32(v, qb);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            xb.q[e] = (int)((uint32_t)(uint8_t)qb.q[4 * e] | ((uint32_t)(uint8_t)qb.q[4 * e + 1] << 8) |
                            ((uint32_t)(uint8_t)qb.q[4 * e + 2] << 16) | ((uint32_t)(uint8_t)qb.q[4 * e + 3] << 24));
        xb.s = h2f_exact(qb.dh);
        xb.sum8 = 8 * qb.sum;
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) xb.x[j] = v[j];
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            a += v[j];
            b += v[16 + j];
        }
        xb.xs0 = a;
        xb.xs1 = b;
        xb.xs = a + b;
    }
}

// Where a lane's 32 elements sit in a chunk buffer whose data starts at byte
// sh (0 for aligned rows), and their dot with the lane's activation.
//
// Q8_0 / Q4_0: the lane's block starts at byte b = sh + BB*lane.  Its fp16
// scale is the halfword b/2 (b is even: blocks and rows have even lengths);
// its quants start at b + 2, which is dword-aligned when b % 4 == 2 and 2
// bytes into a dword otherwise.  Reading dwords from `first` and taking
// alignbyte(dw[k+1], dw[k], shift) gives the k-th quant dword in both cases
// with one instruction and no branch.
template <int QT>
struct Lane {
    uint32_t half, first, shift;

    __device__ __forceinline__ void at(int lane, uint32_t sh) {
        const uint32_t b = sh + (uint32_t)lane * Fmt<QT>::kUnitBytes;
        const bool odd = (b & 2u) != 0;
        half = b >> 1;
        first = (b >> 2) + (odd ? 1u : 0u);
        shift = odd ? 0u : 2u;
    }

    //   Q8_0: d * sum_j q_j x_j with fp32 FMAs;
    //   Q4_0: dw*dx*(float)isum, isum the exact integer dot.
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        const float d = h2f(reinterpret_cast<const uint16_t*>(buf)[half]);
        const uint32_t* p = buf + first;
        if (QT == L3P_Q8_0) {
            uint32_t dw[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) dw[k] = p[k];
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t q = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], shift);
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
                const uint32_t q = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], shift);
                isum = __builtin_amdgcn_sdot4((int)(q & 0x0f0f0f0fu), xb.q[k], isum, false);
                isum = __builtin_amdgcn_sdot4((int)((q >> 4) & 0x0f0f0f0fu), xb.q[4 + k], isum, false);
            }
            return d * xb.s * (float)isum;
        }
    }
};

// Q4_K super-block {fp16 d, dmin; u8 scales[12]; u8 qs[128]} (c:157-162),
// 144 B at byte 144*sb of the buffer (16-byte aligned).  Lane = sub-block
// j = lane % 8 of super-block sb = lane / 8: the low (j even) or high (j odd)
// nibbles of qs[32*(j/2) .. +32].  High nibbles are used in place, masked,
// as 16*q, and the sum is scaled back by 1/16 (exact).
template <>
struct Lane<L3P_Q4_K> {
    uint32_t hdr;    // dword index of {d, dmin, scales[12]}
    uint32_t qs;     // dword index of the lane's 32 quant bytes
    uint32_t mask;   // 0x0f0f0f0f or 0xf0f0f0f0
    uint32_t bs;     // bit offset of scale byte j % 4 within its dword
    float fs;        // 1 or 1/16
    bool hi;         // j >= 4

    __device__ __forceinline__ void at(int lane, uint32_t /*sh: always 0*/) {
        const uint32_t sb = (uint32_t)lane >> 3, j = (uint32_t)lane & 7u;
        hdr = 36u * sb;
        qs = hdr + 4u + 8u * (j >> 1);
        mask = (j & 1u) ? 0xf0f0f0f0u : 0x0f0f0f0fu;
        fs = (j & 1u) ? 0.0625f : 1.0f;
        bs = 8u * (j & 3u);
        hi = j >= 4u;
    }

    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        // dword reads (merged into ds_read_b128 by the compiler): a uint4
        // read here makes the compiler wait for every copy in flight
        uint4 h;
        h.x = buf[hdr];
        h.y = buf[hdr + 1];
        h.z = buf[hdr + 2];
        h.w = buf[hdr + 3];
        const float d = h2f(h.x), dmin = h2f(h.x >> 16);
        // get_scale_min_k4 (c:705-714) for sub-block j, from bytes s[j%4] (in
        // h.y), s[j%4+4] (h.z) and s[j%4+8] (h.w), as bit-field extracts and
        // selects (no divergent branch):
        //   j < 4:  sc = s[j] & 63,                          m = s[j+4] & 63
        //   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4,  m = (s[j+4] >> 4) | (s[j] >> 6) << 4
        const uint32_t sc = __builtin_amdgcn_ubfe(hi ? h.w : h.y, bs, hi ? 4u : 6u) |
                            (hi ? __builtin_amdgcn_ubfe(h.y, bs + 6u, 2u) << 4 : 0u);
        const uint32_t mn = __builtin_amdgcn_ubfe(hi ? h.w : h.z, hi ? bs + 4u : bs, hi ? 4u : 6u) |
                            (hi ? __builtin_amdgcn_ubfe(h.z, bs + 6u, 2u) << 4 : 0u);
        uint32_t qw[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) qw[k] = buf[qs + k];
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t q = qw[k] & mask;
            s0 = fmaf((float)(q & 0xffu), xb.x[4 * k], s0);
            s1 = fmaf((float)((q >> 8) & 0xffu), xb.x[4 * k + 1], s1);
            s2 = fmaf((float)((q >> 16) & 0xffu), xb.x[4 * k + 2], s2);
            s3 = fmaf((float)(q >> 24), xb.x[4 * k + 3], s3);
        }
        const float s = ((s0 + s1) + (s2 + s3)) * fs;
        return (d * (float)sc) * s - (dmin * (float)mn) * xb.xs;
    }
};

// Q6_K super-block {u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d}
// (c:190-195), 210 B at byte base = sh + 210*sb of the buffer (even).  Lane
// = quarter g = lane % 4 of half h = (lane / 4) % 2 of super-block
// sb = lane / 8, i.e. elements 128h + 32g + e, e < 32 (c:873-904):
//   u_e = nibble (g / 2 ? high : low) of ql[64h + 32(g%2) + e]
//         | ((qh[32h + e] >> 2g) & 3) << 4,   q_e = u_e - 32,
//   scale sc[8h + 2g + e/16].
// Each quant dword is one v_alignbit from a pair of buffer dwords: the ql
// stream is read from bit 8*pos + 4*(g/2) (nibble at bits 0..3 of each
// byte), the qh stream from bit 8*pos + 2g - 4 (code bits at 4..5), so
// u = (ql' & 0x0f) | (qh' & 0x30) per byte.
template <>
struct Lane<L3P_Q6_K> {
    uint32_t qlf, qln;   // first dword and bit offset of the ql stream
    uint32_t qhf, qhn;   // same for qh
    uint32_t sch, dh;    // halfword indices of {sc[8h+2g], sc[8h+2g+1]} and d

    __device__ __forceinline__ void at(int lane, uint32_t sh) {
        const uint32_t sb = (uint32_t)lane >> 3, h = ((uint32_t)lane >> 2) & 1u, g = (uint32_t)lane & 3u;
        const uint32_t base = sh + 210u * sb;
        const uint32_t pl = 8u * (base + 64u * h + 32u * (g & 1u)) + 4u * (g >> 1);
        const uint32_t ph = 8u * (base + 128u + 32u * h) + 2u * g - 4u;
        qlf = pl >> 5;
        qln = pl & 31u;
        qhf = ph >> 5;
        qhn = ph & 31u;
        sch = (base + 192u + 8u * h + 2u * g) >> 1;
        dh = (base + 208u) >> 1;
    }

    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        uint32_t l[9], hb[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            l[k] = buf[qlf + k];
            hb[k] = buf[qhf + k];
        }
        const uint16_t* hw = reinterpret_cast<const uint16_t*>(buf);
        const uint32_t scw = hw[sch];
        const float d = h2f(hw[dh]);
        float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t ql = __builtin_amdgcn_alignbit(l[k + 1], l[k], qln);
            const uint32_t qh = __builtin_amdgcn_alignbit(hb[k + 1], hb[k], qhn);
            const uint32_t u = (ql & 0x0f0f0f0fu) | (qh & 0x30303030u);
            if (k < 4) {
                a0 = fmaf((float)(u & 0xffu), xb.x[4 * k], a0);
                a1 = fmaf((float)((u >> 8) & 0xffu), xb.x[4 * k + 1], a1);
                a0 = fmaf((float)((u >> 16) & 0xffu), xb.x[4 * k + 2], a0);
                a1 = fmaf((float)(u >> 24), xb.x[4 * k + 3], a1);
            } else {
                b0 = fmaf((float)(u & 0xffu), xb.x[4 * k], b0);
                b1 = fmaf((float)((u >> 8) & 0xffu), xb.x[4 * k + 1], b1);
                b0 = fmaf((float)((u >> 16) & 0xffu), xb.x[4 * k + 2], b0);
                b1 = fmaf((float)(u >> 24), xb.x[4 * k + 3], b1);
            }
        }
        const float sc0 = (float)(int8_t)(scw & 0xffu), sc1 = (float)(int8_t)(scw >> 8);
        return d * (sc0 * ((a0 + a1) - 32.0f * xb.xs0) + sc1 * ((b0 + b1) - 32.0f * xb.xs1));
    }
};

// Eight dwords of a byte stream starting at bit `pos` of buf: nine aligned
// dword reads and a funnel shift each (any byte or bit alignment).
__device__ __forceinline__ void bit_window8(const uint32_t* buf, uint32_t pos, uint32_t (&w)[8]) {
    const uint32_t f = pos >> 5, n = pos & 31u;
    uint32_t d[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) d[k] = buf[f + k];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], n);
}

// Four bits b0..b3 of n -> 0x10 in the bytes whose bit is set: the fifth
// bit of four Q5 codes (n * 0x204081 puts bit i at bit 8i, masked).
__device__ __forceinline__ uint32_t spread4(uint32_t n) {
    return (((n & 15u) * 0x00204081u) & 0x01010101u) << 4;
}

// exact isum of the four low / four high nibble dwords of a 32-block
// against the Q8_0 activation quants
__device__ __forceinline__ int nib_dot(const uint32_t (&lo)[4], const uint32_t (&hi)[4], const XBlock& xb, int isum) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        isum = __builtin_amdgcn_sdot4((int)lo[k], xb.q[k], isum, false);
        isum = __builtin_amdgcn_sdot4((int)hi[k], xb.q[4 + k], isum, false);
    }
    return isum;
}

// Q4_1 {fp16 d, m; u8 qs[16]} (c:140-145): the lane's block at byte
// b = sh + 20*lane (4-aligned: rows and chunks start 4-aligned).  Per block
// the reference's dw*dx*isum + mw*dx*xsum with isum = sum xq*u, xsum = sum xq
// (vec_dot_q4_1_q8_0, c:1646-1665).
template <>
struct Lane<L3P_Q4_1> {
    uint32_t hdr;
    __device__ __forceinline__ void at(int lane, uint32_t sh) { hdr = (sh + 20u * (uint32_t)lane) >> 2; }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        const uint32_t dm = buf[hdr];
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = buf[hdr + 1 + k];
            lo[k] = q & 0x0f0f0f0fu;
            hi[k] = (q >> 4) & 0x0f0f0f0fu;
        }
        const int isum = nib_dot(lo, hi, xb, 0);
        return h2f(dm) * xb.s * (float)isum + h2f(dm >> 16) * xb.s * (float)(xb.sum8 / 8);
    }
};

// Q5_0 {fp16 d; u8 qh[4]; u8 qs[16]} (c:147-151): block at byte
// b = sh + 22*lane (even).  Code u_j = nibble | bit j of qh << 4; per block
// dw*dx*isum with isum = sum xq*(u - 16) (vec_dot_q5_0_q8_0, c:1668-1690).
template <>
struct Lane<L3P_Q5_0> {
    uint32_t half, pos;   // halfword of d; bit position of qh (qs follows)
    __device__ __forceinline__ void at(int lane, uint32_t sh) {
        const uint32_t b = sh + 22u * (uint32_t)lane;
        half = b >> 1;
        pos = 8u * (b + 2u);
    }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        const uint32_t f = pos >> 5, n = pos & 31u;
        uint32_t d[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) d[k] = buf[f + k];
        const uint32_t qh = __builtin_amdgcn_alignbit(d[1], d[0], n);
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = __builtin_amdgcn_alignbit(d[k + 2], d[k + 1], n);
            lo[k] = (q & 0x0f0f0f0fu) | spread4(qh >> (4 * k));
            hi[k] = ((q >> 4) & 0x0f0f0f0fu) | spread4(qh >> (16 + 4 * k));
        }
        const int isum = nib_dot(lo, hi, xb, -2 * xb.sum8);
        return h2f(reinterpret_cast<const uint16_t*>(buf)[half]) * xb.s * (float)isum;
    }
};

// Q5_1 {fp16 d, m; u8 qh[4]; u8 qs[16]} (c:153-158): block at byte
// b = sh + 24*lane (8-aligned).  dw*dx*isum + mw*dx*xsum with isum = sum xq*u
// (vec_dot_q5_1_q8_0, c:1693-1717).
template <>
struct Lane<L3P_Q5_1> {
    uint32_t hdr;
    __device__ __forceinline__ void at(int lane, uint32_t sh) { hdr = (sh + 24u * (uint32_t)lane) >> 2; }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        const uint32_t dm = buf[hdr], qh = buf[hdr + 1];
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = buf[hdr + 2 + k];
            lo[k] = (q & 0x0f0f0f0fu) | spread4(qh >> (4 * k));
            hi[k] = ((q >> 4) & 0x0f0f0f0fu) | spread4(qh >> (16 + 4 * k));
        }
        const int isum = nib_dot(lo, hi, xb, 0);
        return h2f(dm) * xb.s * (float)isum + h2f(dm >> 16) * xb.s * (float)(xb.sum8 / 8);
    }
};

// IQ4_NL {fp16 d; u8 qs[16]} (c:197-201): the Q4_0 layout, nibbles indexing
// the 16-entry code book (c:204-206); dw*dx*isum with isum = sum xq*table[u]
// (vec_dot_iq4_nl_q8_0, c:1994-2011).  Four nibble bytes map through the
// table with two byte permutes (entries 0..7 and 8..15) and a select on
// bit 3.
template <>
struct Lane<L3P_IQ4_NL> : Lane<L3P_Q4_0> {
    static __device__ __forceinline__ uint32_t lookup(uint32_t nib) {
        const uint32_t sel = nib & 0x07070707u;
        const uint32_t a = __builtin_amdgcn_perm(0xF6EADDCFu, 0xBFAD9881u, sel);   // -127 -104 -83 -65 | -49 -35 -22 -10
        const uint32_t b = __builtin_amdgcn_perm(0x71594535u, 0x26190D01u, sel);   //    1   13  25  38 |  53  69  89 113
        const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xffu;
        return (a & ~m) | (b & m);
    }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        const float d = h2f(reinterpret_cast<const uint16_t*>(buf)[half]);
        const uint32_t* p = buf + first;
        uint32_t dw[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) dw[k] = p[k];
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], shift);
            lo[k] = lookup(q & 0x0f0f0f0fu);
            hi[k] = lookup((q >> 4) & 0x0f0f0f0fu);
        }
        return d * xb.s * (float)nib_dot(lo, hi, xb, 0);
    }
};

// fp32 dot of four packed unsigned byte codes with four activations
__device__ __forceinline__ void ubyte_fma(uint32_t u, const float* x, float& s0, float& s1) {
    s0 = fmaf((float)(u & 0xffu), x[0], s0);
    s1 = fmaf((float)((u >> 8) & 0xffu), x[1], s1);
    s0 = fmaf((float)((u >> 16) & 0xffu), x[2], s0);
    s1 = fmaf((float)(u >> 24), x[3], s1);
}

// Q2_K super-block {u8 scales[16]; u8 qs[64]; fp16 d, dmin} (c:165-170), 84 B
// at byte base = sh + 84*sb of the buffer (4-aligned).  Lane = 32-element
// slice k = lane % 8 of super-block sb = lane / 8: groups 2k and 2k+1 of 16,
// 2-bit codes at shift 2j of qs[32*half + l] (half = k / 4, j = k % 4), scale
// byte scales[g] = (min << 4) | scale (dequantize_row_q2_K, c:748-784).
// Each weight is formed as the reference forms it, w = dl*u - ml with
// dl = d*sc and ml = dmin*m (dl*u is exact: 11 + 4 + 2 bits, so fmaf gives
// the reference's value), and the dot is sum w*x in fp32.  The factored form
// dl*sum u x - ml*sum x cancels: with 2-bit codes the two terms are close,
// and their rounding errors flip Q8_0 roundings of K and V that the
// reference does not flip.
template <>
struct Lane<L3P_Q2_K> {
    uint32_t qs, sch, dd, sj;   // dword of the codes, halfword of the two scale bytes, dword of {d, dmin}, 2j
    __device__ __forceinline__ void at(int lane, uint32_t sh) {
        const uint32_t sb = (uint32_t)lane >> 3, k = (uint32_t)lane & 7u;
        const uint32_t base = sh + 84u * sb;
        qs = (base + 16u + 32u * (k >> 2)) >> 2;
        sch = (base + 2u * k) >> 1;
        dd = (base + 80u) >> 2;
        sj = 2u * (k & 3u);
    }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = buf[qs + i];
        const uint32_t scw = reinterpret_cast<const uint16_t*>(buf)[sch];
        const uint32_t dm = buf[dd];
        const float d = h2f(dm), dmin = h2f(dm >> 16);
        const float dl[2] = {d * (float)(scw & 15u), d * (float)((scw >> 8) & 15u)};
        const float ml[2] = {dmin * (float)((scw >> 4) & 15u), dmin * (float)((scw >> 12) & 15u)};
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = (w[i] >> sj) & 0x03030303u;
            const float a = dl[i >> 2], m = ml[i >> 2];
            s0 = fmaf(fmaf(a, (float)(u & 0xffu), -m), xb.x[4 * i], s0);
            s1 = fmaf(fmaf(a, (float)((u >> 8) & 0xffu), -m), xb.x[4 * i + 1], s1);
            s2 = fmaf(fmaf(a, (float)((u >> 16) & 0xffu), -m), xb.x[4 * i + 2], s2);
            s3 = fmaf(fmaf(a, (float)(u >> 24), -m), xb.x[4 * i + 3], s3);
        }
        return (s0 + s1) + (s2 + s3);
    }
};

// Q3_K super-block {u8 hmask[32]; u8 qs[64]; u8 scales[12]; fp16 d}
// (c:172-178), 110 B at byte base = sh + 110*sb (even).  Lane slice k as in
// Q2_K; element l of group 2k + (l >= 16) has code v = u | h << 2 with u the
// 2 bits at shift 2j of qs[32*half + l] and h bit 4*half + j of hmask[l],
// value v - 4, and the 6-bit scale s_g (low 4 bits from byte g or the high
// nibble of byte g - 8, high 2 bits from byte 8 + g%4 at bit 2*(g/4))
// (dequantize_row_q3_K, c:786-832).  As for Q2_K, each weight is the
// reference's exact value w = dl*(v - 4), dl = d*(s - 32) (11 + 6 + 3 bits),
// formed as fmaf(dl, v, -4 dl), and the dot is sum w*x in fp32.
template <>
struct Lane<L3P_Q3_K> {
    uint32_t qpos, hpos, spos, dh;   // bit positions of qs, hmask, scales; halfword of d
    uint32_t sj, hr, hl;             // 2j; hmask bit 4*half + j moved to bit 2 by >> hr << hl
    uint32_t olo, ohi;               // bit offsets of group a's low nibble and high bits in the scale bytes
    __device__ __forceinline__ void at(int lane, uint32_t sh) {
        const uint32_t sb = (uint32_t)lane >> 3, k = (uint32_t)lane & 7u;
        const uint32_t base = sh + 110u * sb, half = k >> 2, j = k & 3u, hb = 4u * half + j;
        qpos = 8u * (base + 32u + 32u * half);
        hpos = 8u * base;
        spos = 8u * (base + 96u);
        dh = (base + 108u) >> 1;
        sj = 2u * j;
        hr = hb >= 2u ? hb - 2u : 0u;
        hl = hb >= 2u ? 0u : 2u - hb;
        olo = k < 4u ? 16u * k : 16u * (k - 4u) + 4u;
        ohi = 64u + 16u * (k & 1u) + 2u * (k >> 1);
    }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        uint32_t q[8], h[8];
        bit_window8(buf, qpos, q);
        bit_window8(buf, hpos, h);
        const uint32_t f = spos >> 5, n = spos & 31u;
        const uint32_t s0 = __builtin_amdgcn_alignbit(buf[f + 1], buf[f], n);
        const uint32_t s1 = __builtin_amdgcn_alignbit(buf[f + 2], buf[f + 1], n);
        const uint32_t s2 = __builtin_amdgcn_alignbit(buf[f + 3], buf[f + 2], n);
        const float d = h2f(reinterpret_cast<const uint16_t*>(buf)[dh]);
        const uint32_t sl = olo < 32u ? s0 : s1;
        const uint32_t ol = olo & 31u, oh = ohi - 64u;
        const int sa = (int)(__builtin_amdgcn_ubfe(sl, ol, 4u) | (__builtin_amdgcn_ubfe(s2, oh, 2u) << 4)) - 32;
        const int sb = (int)(__builtin_amdgcn_ubfe(sl, ol + 8u, 4u) | (__builtin_amdgcn_ubfe(s2, oh + 8u, 2u) << 4)) - 32;
        const float dl[2] = {d * (float)sa, d * (float)sb};
        float t0 = 0.0f, t1 = 0.0f, t2 = 0.0f, t3 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = ((q[i] >> sj) & 0x03030303u) | (((h[i] >> hr) << hl) & 0x04040404u);
            const float a = dl[i >> 2], m = -4.0f * dl[i >> 2];
            t0 = fmaf(fmaf(a, (float)(v & 0xffu), m), xb.x[4 * i], t0);
            t1 = fmaf(fmaf(a, (float)((v >> 8) & 0xffu), m), xb.x[4 * i + 1], t1);
            t2 = fmaf(fmaf(a, (float)((v >> 16) & 0xffu), m), xb.x[4 * i + 2], t2);
            t3 = fmaf(fmaf(a, (float)(v >> 24), m), xb.x[4 * i + 3], t3);
        }
        return (t0 + t1) + (t2 + t3);
    }
};

// Q5_K super-block {fp16 d, dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]}
// (c:180-187), 176 B at byte 176*sb (16-byte aligned).  Lane = sub-block
// k = lane % 8: code = nibble of qs[32*(k/2) + l] (low for even k) + 16 * bit
// k of qh[l], with the Q4_K 6-bit scale and min k:
//   (d*sc)*sum q x - (dmin*m)*sum x   (dequantize_row_q5_K, c:834-871).
template <>
struct Lane<L3P_Q5_K> {
    uint32_t hdr, qh, qs, ns, kb, bs;
    bool hi;
    __device__ __forceinline__ void at(int lane, uint32_t /*sh: always 0*/) {
        const uint32_t sb = (uint32_t)lane >> 3, k = (uint32_t)lane & 7u;
        hdr = 44u * sb;
        qh = hdr + 4u;
        qs = hdr + 12u + 8u * (k >> 1);
        ns = 4u * (k & 1u);
        kb = k;
        bs = 8u * (k & 3u);
        hi = k >= 4u;
    }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        uint4 h;   // dword reads (merged by the compiler), as in Lane<Q4_K>
        h.x = buf[hdr];
        h.y = buf[hdr + 1];
        h.z = buf[hdr + 2];
        h.w = buf[hdr + 3];
        const float d = h2f(h.x), dmin = h2f(h.x >> 16);
        const uint32_t sc = __builtin_amdgcn_ubfe(hi ? h.w : h.y, bs, hi ? 4u : 6u) |
                            (hi ? __builtin_amdgcn_ubfe(h.y, bs + 6u, 2u) << 4 : 0u);
        const uint32_t mn = __builtin_amdgcn_ubfe(hi ? h.w : h.z, hi ? bs + 4u : bs, hi ? 4u : 6u) |
                            (hi ? __builtin_amdgcn_ubfe(h.z, bs + 6u, 2u) << 4 : 0u);
        uint32_t qw[8], hw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            qw[i] = buf[qs + i];
            hw[i] = buf[qh + i];
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = ((qw[i] >> ns) & 0x0f0f0f0fu) | (((hw[i] >> kb) & 0x01010101u) << 4);
            ubyte_fma(q, xb.x + 4 * i, s0, s1);
        }
        return (d * (float)sc) * (s0 + s1) - (dmin * (float)mn) * xb.xs;
    }
};

// F16 / BF16 rows: the lane's 32 values are the 64 bytes at 64*lane, two per
// dword, converted exactly and summed as fp32 products (vec_dot_f16 /
// vec_dot_bf16, c:1467-1485, sum in another order).
template <int QT>
struct LaneHalf {
    uint32_t first;
    __device__ __forceinline__ void at(int lane, uint32_t /*sh: always 0*/) { first = 16u * (uint32_t)lane; }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        uint32_t w[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = buf[first + i];
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            float v[4];
            if (QT == L3P_F16) {
                v[0] = h2f(w[i]); v[1] = h2f(w[i] >> 16); v[2] = h2f(w[i + 1]); v[3] = h2f(w[i + 1] >> 16);
            } else {
                v[0] = __uint_as_float(w[i] << 16); v[1] = __uint_as_float(w[i] & 0xffff0000u);
                v[2] = __uint_as_float(w[i + 1] << 16); v[3] = __uint_as_float(w[i + 1] & 0xffff0000u);
            }
            s0 = fmaf(v[0], xb.x[2 * i], s0);
            s1 = fmaf(v[1], xb.x[2 * i + 1], s1);
            s2 = fmaf(v[2], xb.x[2 * i + 2], s2);
            s3 = fmaf(v[3], xb.x[2 * i + 3], s3);
        }
        return (s0 + s1) + (s2 + s3);
    }
};
template <> struct Lane<L3P_F16> : LaneHalf<L3P_F16> {};
template <> struct Lane<L3P_BF16> : LaneHalf<L3P_BF16> {};

// F32 rows: the lane's 32 values are the 128 bytes at 128*lane (vec_dot_f32,
// c:1487-1494, sum in another order).
template <>
struct Lane<L3P_F32> {
    uint32_t first;
    __device__ __forceinline__ void at(int lane, uint32_t /*sh: always 0*/) { first = 32u * (uint32_t)lane; }
    __device__ __forceinline__ float dot(const uint32_t* buf, const XBlock& xb) const {
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            s0 = fmaf(__uint_as_float(buf[first + i]), xb.x[i], s0);
            s1 = fmaf(__uint_as_float(buf[first + i + 1]), xb.x[i + 1], s1);
            s2 = fmaf(__uint_as_float(buf[first + i + 2]), xb.x[i + 2], s2);
            s3 = fmaf(__uint_as_float(buf[first + i + 3]), xb.x[i + 3], s3);
        }
        return (s0 + s1) + (s2 + s3);
    }
};

// RG: built with row ranges (a.rpw > 0); kernels without them carry none of
// their per-chunk branches (measured 3-5% faster at the standalone C1-C3
// shapes and 0.7% on the Llama-3-8B decode step on MI355X).
template <int QT, int G, int NB, bool PAIR, bool UA, bool POST, bool RG = false>
__global__ void __launch_bounds__(POST ? 512 : 1024) gemv_kernel(GemvArgs a) {
    constexpr int CB = Fmt<QT>::kChunkBytes;
    constexpr int CDW = Fmt<QT>::kBufBytes / 4;
    constexpr int CI = Fmt<QT>::kCI;
    constexpr int NOUT = PAIR ? G / 2 : G;
    // the normed residual hand-over (xw / ssp out, ss in) is for one-segment
    // GEMVs without the residual update; launch_gemv rejects other mixes, and
    // leaving its registers out of the pair and residual-update kernels keeps
    // their prologue loads clear of the register allocator
    constexpr bool kConsume = !PAIR && !POST;
    constexpr bool kProduce = !PAIR && !POST;
    extern __shared__ __align__(16) uint32_t lds[];
    const int t = threadIdx.x, lane = t & 63, nw = blockDim.x >> 6;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nb = a.cols >> 5;   // 32-element lane slots of a row
    const uint32_t rb = row_bytes<QT>(a.cols);
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
    // row ranges (rpw > 0, never in pair mode): this workgroup's rows
    const bool ranges = RG && !PAIR && a.rpw > 0;
    cc.rbeg = (int)blockIdx.x * a.rpw;
    cc.nmine = ranges ? max(0, min(a.rpw, a.rows_total - cc.rbeg)) : -1;
    cc.rb = rb;
    cc.coff = (uint32_t)w * (uint32_t)CB;
    const int nbytes = (int)min((uint32_t)CB, rb - cc.coff);   // this wave's chunk length
    const DmaLane dl = dma_lane<QT>(lane, nbytes);
    // copy row-chunk k of the sequence into ring slot `slot`
    auto issue = [&](int k, int slot) {
        const uint8_t* src;
        chunk_src<G, PAIR, RG>(cc, k, src);
        if (UA) {
            const uint32_t sh = (uint32_t)(uintptr_t)src & 15u;
            chunk_dma<QT>(ring + slot * CDW, src - sh, dma_lane<QT>(lane, (int)sh + nbytes));
        } else {
            chunk_dma<QT>(ring + slot * CDW, src, dl);
        }
    };
    float* red = reinterpret_cast<float*>(lds + (size_t)nw * NB * CDW);   // [2][nw][G]
    float* ssred = red + 2 * nw * G;                                      // [nw]
    float* ssy = ssred + nw;                                              // [nw] (post norm)
    float* out_lds = ssy + nw;                                            // [groups of this WG][NOUT]

    // ---- this lane's activation block, the norm weights and the residual
    // update's inputs: issued before the weight copies, waited for after them
    // without waiting for the copies (see load8_async).  Lanes past the row
    // load the last block and drop it.
    const int blk = w * 64 + lane;
    const bool active = blk < nb;
    const int lblk = active ? blk : nb - 1;
    f32x4 xq[8], nq[8], yq[8], pq[8], sq[4];
    load8_async(xq, a.x + 32 * lblk);
    if (a.norm) load8_async(nq, a.norm + 32 * lblk);
    if (POST) {
        load8_async(yq, a.post_y + 32 * lblk);
        load8_async(pq, a.post_w + 32 * lblk);
    }
    // the producer's partial sums of squares (zero past its workgroups), 256
    // per load; a residual-add producer's norm weights for its first output
    if (kConsume && a.ss) {
#pragma unroll
        for (int i = 0; i < kMaxSsParts / 256; ++i)
            if (i < a.ss_loads)
                asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(sq[i]) : "v"(a.ss + 4 * lane + 256 * i));
    }
    const int ngroups_mine =
        ranges ? (cc.nmine + G - 1) / G
               : (a.ngroups > (int)blockIdx.x ? (a.ngroups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0);
    const int nout_mine = ranges ? cc.nmine : ngroups_mine * NOUT;   // output rows of this workgroup
    float wfirst = 0.0f;   // xw_w at this thread's first output row (the epilogue's j = t)
    if (kProduce && a.xw && t < nout_mine) {
        const int gi = ranges ? cc.rbeg + t : ((int)blockIdx.x) * G + t % NOUT + (t / NOUT) * (int)gridDim.x * G;
        asm volatile("global_load_dword %0, %1, off" : "=v"(wfirst) : "v"(a.xw_w + min(gi, a.rows_total - 1)));
    }

    // ---- weight copies: the first NB-1 chunks of this workgroup's sequence,
    // CI instructions each.  nk = number of row-chunks this wave copies; with
    // row ranges the slots of the last group past nk are neither copied nor
    // waited for (their dots read a stale buffer and are dropped).
    const int nk = ranges ? cc.nmine : ngroups_mine * G;
#pragma unroll
    for (int b = 0; b < NB - 1; ++b)
        if (b < nk) issue(b, b);
    wait_prologue<NB - 1, CI>(nk);
    pin8(xq);
    if (a.norm) pin8(nq);
    if (POST) {
        pin8(yq);
        pin8(pq);
    }
    asm volatile("" : "+v"(wfirst));
    if (kConsume && a.ss) {
#pragma unroll
        for (int i = 0; i < kMaxSsParts / 256; ++i)
            if (i < a.ss_loads) asm volatile("" : "+v"(sq[i]));
    }
    float v[32];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        v[4 * e] = active ? xq[e].x : 0.0f;
        v[4 * e + 1] = active ? xq[e].y : 0.0f;
        v[4 * e + 2] = active ? xq[e].z : 0.0f;
        v[4 * e + 3] = active ? xq[e].w : 0.0f;
    }

    // x := x + post_w * (r_y * post_y) (rmsnorm_add_kernel's arithmetic), the
    // same in every workgroup; the first workgroup stores it
    if (POST) {
        float sy = 0.0f;
        if (active) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sy += yq[e].x * yq[e].x;
                sy += yq[e].y * yq[e].y;
                sy += yq[e].z * yq[e].z;
                sy += yq[e].w * yq[e].w;
            }
        }
        sy = wave_sum(sy);
        if (lane == 0) ssy[w] = sy;
        lds_sync();
        sy = 0.0f;
        for (int i = 0; i < nw; ++i) sy += ssy[i];
        const float ry = 1.0f / sqrtf(sy * a.inv_n + a.eps);
        if (active) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[4 * e] = v[4 * e] + pq[e].x * (ry * yq[e].x);
                v[4 * e + 1] = v[4 * e + 1] + pq[e].y * (ry * yq[e].y);
                v[4 * e + 2] = v[4 * e + 2] + pq[e].z * (ry * yq[e].z);
                v[4 * e + 3] = v[4 * e + 3] + pq[e].w * (ry * yq[e].w);
            }
            if (blockIdx.x == 0) {
                float4* op = reinterpret_cast<float4*>(a.post_out + 32 * blk);
#pragma unroll
                for (int e = 0; e < 8; ++e) op[e] = make_float4(v[4 * e], v[4 * e + 1], v[4 * e + 2], v[4 * e + 3]);
            }
        }
    }

    // ---- optional RMSNorm.  Every block of x belongs to exactly one lane, so
    // ss = sum over lanes of the lane's 32 squares, then over lanes and waves
    // in a fixed order: the same value in every workgroup.  For fp32
    // activations the GEMV is linear in x, so the lanes take w[j] * x[j] and
    // the row totals are scaled by r after the first group's cross-wave sum:
    // nothing here waits for the other waves.  Q4_0 quantizes w[j] * (r *
    // x[j]) exactly as the reference does, so it forms r first.
    constexpr bool kLateScale = !q8_act<QT>();
    if (a.norm) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) ss += v[j] * v[j];
        ss = wave_sum(ss);
        if (lane == 0) ssred[w] = ss;
        float r = 1.0f;
        if (!kLateScale) {
            lds_sync();
            ss = 0.0f;
            for (int i = 0; i < nw; ++i) ss += ssred[i];
            r = 1.0f / sqrtf(ss * a.inv_n + a.eps);
        }
        if (active) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (kLateScale) {
                    v[4 * e] = nq[e].x * v[4 * e];
                    v[4 * e + 1] = nq[e].y * v[4 * e + 1];
                    v[4 * e + 2] = nq[e].z * v[4 * e + 2];
                    v[4 * e + 3] = nq[e].w * v[4 * e + 3];
                } else {
                    v[4 * e] = nq[e].x * (r * v[4 * e]);
                    v[4 * e + 1] = nq[e].y * (r * v[4 * e + 1]);
                    v[4 * e + 2] = nq[e].z * (r * v[4 * e + 2]);
                    v[4 * e + 3] = nq[e].w * (r * v[4 * e + 3]);
                }
            }
        }
    }
    float rscale = 1.0f;   // late RMSNorm scale of the row totals (threads t < NOUT)
    float rss = 1.0f;      // the same from a producer's partial sums
    XBlock xb;
    prepare_block<QT>(v, xb);
    Lane<QT> ln;
    ln.at(lane, 0u);

    // ---- row loop: G rows per group, chunk k = gl*G + i of this WG's sequence
    for (int gl = 0; gl < ngroups_mine; ++gl) {
        float acc[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int k = gl * G + i;
            // refill first: chunk k+NB-1 goes to the buffer of chunk k-1, whose
            // LDS reads finished in the previous step, so NB-1 copies stay in
            // flight while chunk k is computed
            const int kn = k + NB - 1;
            if (kn < nk) issue(kn, kn % NB);
            // chunk k is in LDS once only the younger chunks' copies remain:
            // NB-1 of them in steady state, fewer near the end of the sequence
            wait_chunk<NB - 1, CI>(nk - 1 - k);
            const uint8_t* src;
            const bool real = chunk_src<G, PAIR, RG>(cc, k, src);
            if (UA) ln.at(lane, (uint32_t)(uintptr_t)src & 15u);
            // every lane reads inside the buffer, so the dot runs unconditionally
            // and lanes past the row or rows past the matrix drop their value
            float dv = ln.dot(ring + (k % NB) * CDW, xb);
            // pin the dot here: left alone, the compiler sinks every dot of the
            // group to its end and keeps all their quants live in registers
            asm volatile("" : "+v"(dv));
            const float d = (real && active) ? dv : 0.0f;
            wait_lgkm();   // this chunk's LDS reads are done before its buffer is refilled
            acc[i] = d;
        }
        // group done: wave totals -> LDS -> sum over the chunk waves in order
        if (kConsume && a.ss && gl == 0) {   // x arrived normed but for the scale: r from the partial sums, in a fixed order
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < kMaxSsParts / 256; ++i) {
                if (i < a.ss_loads) {
                    const int e = 256 * i + 4 * lane;
                    ss += e < a.n_ss ? sq[i].x : 0.0f;
                    ss += e + 1 < a.n_ss ? sq[i].y : 0.0f;
                    ss += e + 2 < a.n_ss ? sq[i].z : 0.0f;
                    ss += e + 3 < a.n_ss ? sq[i].w : 0.0f;
                }
            }
            ss = wave_sum(ss);
            rss = 1.0f / sqrtf(ss * a.inv_n + a.eps);
        }
        float* rd = red + (gl & 1) * nw * G;
        const float tot = xreduce<G>(acc, lane);
        if ((lane & ((64 / G) - 1)) == 0) rd[w * G + rowof<G>(lane)] = tot;
        lds_sync();
        if (t < NOUT) {
            if (kLateScale && a.norm && gl == 0) {   // every wave's ss is in LDS by now
                float ss = 0.0f;
                for (int i = 0; i < nw; ++i) ss += ssred[i];
                rscale = 1.0f / sqrtf(ss * a.inv_n + a.eps);
            }
            if (kConsume && a.ss && gl == 0) rscale = rss;
            float s0 = 0.0f;
            for (int c = 0; c < nw; ++c) s0 += rd[c * G + t];
            s0 *= rscale;
            float res = s0;
            if (PAIR) {
                float s1 = 0.0f;
                for (int c = 0; c < nw; ++c) s1 += rd[c * G + G / 2 + t];
                s1 *= rscale;
                res = a.epilogue == EPI_GEGLU ? ref_geglu(s0, s1) : ref_swiglu(s0, s1);
            }
            out_lds[gl * NOUT + t] = res;
        }
    }
    // ---- results of this workgroup's groups (every copy has been waited for)
    lds_sync();
    float ssq = 0.0f;   // this thread's sum of its new residuals' squares (xw set)
    for (int j = t; j < nout_mine; j += blockDim.x) {
        const int gk = j / NOUT, i = j % NOUT;
        const int grp = blockIdx.x + gk * gridDim.x;
        if (PAIR) {
            const int row = grp * NOUT + i;
            if (row < a.rows[0]) a.y[0][row] = out_lds[j];
        } else {
            const int gi = ranges ? cc.rbeg + j : grp * G + i;
            if (gi >= a.rows_total) continue;
            int s, row;
            seg_of(a, gi, s, row);
            float* y = a.y[s] + row;
            if (a.epilogue == EPI_ADD) {
                const float nx = *y + out_lds[j];
                *y = nx;
                if (kProduce && a.xw) {   // one segment: gi is the row
                    a.xw[gi] = nx * (j == t ? wfirst : a.xw_w[gi]);
                    ssq += nx * nx;
                }
            } else {
                *y = out_lds[j];
            }
        }
    }
    if (kProduce && a.xw) {   // the workgroup's sum: threads in order within waves, then waves in order
        if (nout_mine <= 64) {   // every output is wave 0's: no barrier
            if (w == 0) {
                ssq = wave_sum(ssq);
                if (lane == 0) a.ssp[blockIdx.x] = ssq;
            }
        } else {
            ssq = wave_sum(ssq);
            if (lane == 0) ssred[w] = ssq;
            lds_sync();
            if (t == 0) {
                float tot = 0.0f;
                for (int i = 0; i < nw; ++i) tot += ssred[i];
                a.ssp[blockIdx.x] = tot;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q8_0 rows of 2048 < cols <= 2560 columns, cols = 256 J (Gemma-2-2B's 2304):
// whole rows per wave.  The chunk-column kernel above gives such a row a
// second wave for its last 256 or 512 columns, and that wave issues a whole
// activation's worth of prologue loads (8 per vector, whatever few lanes
// carry data) and copies its short chunk with as many instructions as a full
// one.  Here one wave streams whole rows, RB = 272 J bytes each, copied with
// ceil(RB / 1024) dwordx4 instructions into a private ring of NB buffers, and lane l
// owns the columns 256 j + 4 l .. 256 j + 4 l + 3 for j < J: an activation
// vector is J coalesced 16-byte loads per lane, a row's dot needs no
// cross-wave sum (there is no barrier in the kernel), and the residual update
// and the RMSNorm of the prologue reduce over the wave alone.  A workgroup is
// one wave, persistent over groups of G rows as in gemv_kernel.
//
// Lane l's four columns of group j lie in block b = 8 j + l / 8, at quant
// bytes 4 (l % 8) .. + 3, i.e. at byte 34 b + 2 + 4 (l % 8) of the row:
// dword-aligned when b is odd and 2 bytes into a dword when b is even (b has
// the parity of l / 8), so one alignbyte of two buffer dwords gives the four
// quants.  The lane's term for the group is d_b * sum q x over its four
// columns (gemv_kernel's d * sum q_j x_j, over four columns instead of 32).
// ---------------------------------------------------------------------------
// dwordx4 copy instructions of a row of J 256-column groups (272 J bytes)
template <int J>
constexpr int wide_ci() { return (17 * J + 63) / 64; }

// Rows of 2304 and 2560 columns.  At 4096 columns, where the chunk-column
// kernel's two waves both carry full chunks, whole rows were slower (Llama-3-8B
// gate|up 23.2 -> 25.3 us, wo 8.1 -> 8.4 us in the decode step on MI355X).
bool wide_cols(int cols) { return cols > kChunkElems && cols <= 2560 && cols % 256 == 0; }

// Lane offsets of a row copy: piece i*64 + lane of the row's RB/16 pieces,
// clamped to the last piece (clamped lanes re-read it and write it past RB in
// the buffer), so every row is exactly CI instructions.
struct WideDma {
    int o[8];   // CI <= 8 (rows of up to 30 groups)
};
template <int CI>
__device__ __forceinline__ WideDma wide_dma(int lane, uint32_t rb) {
    static_assert(CI <= 8, "at most eight copy instructions per row");
    const int last = (int)(rb >> 4) - 1;
    WideDma d;
#pragma unroll
    for (int i = 0; i < CI; ++i) d.o[i] = 16 * min(64 * i + lane, last);
    return d;
}
template <int CI>
__device__ __forceinline__ void wide_copy(uint32_t* dst, const uint8_t* src, const WideDma& d) {
#pragma unroll
    for (int i = 0; i < CI; ++i) __builtin_amdgcn_global_load_lds(src + d.o[i], (lds_void*)(dst + 256 * i), 16, 0, 2);
}

// J untracked 16-byte loads per lane, 256 floats apart (see load8_async)
template <int J>
__device__ __forceinline__ void loadj_async(f32x4 (&q)[J], const float* p) {
#pragma unroll
    for (int j = 0; j < J; ++j) asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(q[j]) : "v"(p + 256 * j));
}
template <int J>
__device__ __forceinline__ void pinj(f32x4 (&q)[J]) {
#pragma unroll
    for (int j = 0; j < J; ++j) asm volatile("" : "+v"(q[j]));
}

template <int J, int G, int NB, bool PAIR, bool POST, int S = 1>
__global__ void __launch_bounds__(64 * S) gemv_wide_kernel(GemvArgs a) {
    static_assert(S == 1 || (!PAIR && !POST), "sliced rows: plain rows only");
    constexpr int NOUT = PAIR ? G / 2 : G;
    constexpr int CI = wide_ci<J>();
    constexpr int BDW = CI * 256;   // dwords per ring buffer
    extern __shared__ __align__(16) uint32_t lds[];
    // S > 1: wave s takes bytes [272 J s, 272 J (s + 1)) of every row (columns
    // [256 J s, 256 J (s + 1))) through its own ring
    const int sl = S > 1 ? (int)(threadIdx.x >> 6) : 0;
    uint32_t* ring = lds + sl * NB * BDW;
    float* xch = reinterpret_cast<float*>(lds + S * NB * BDW);   // [G] row totals (pair epilogue); S > 1: [2][S][G]
    const int lane = threadIdx.x & 63;
    const uint32_t rb = 272u * J;
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
    cc.rbeg = 0;
    cc.nmine = -1;
    cc.rb = rb * S;
    cc.coff = rb * sl;
    const WideDma dl = wide_dma<CI>(lane, rb);
    auto issue = [&](int k, int slot) {
        const uint8_t* src;
        chunk_src<G, PAIR>(cc, k, src);
        wide_copy<CI>(ring + slot * BDW, src, dl);
    };

    // ---- the lane's activation columns, norm weights and residual-update
    // inputs, issued before the weight copies and waited for without them
    f32x4 xq[J], nq[J], yq[J], pq[J];
    loadj_async<J>(xq, a.x + 256 * J * sl + 4 * lane);
    if (a.norm) loadj_async<J>(nq, a.norm + 4 * lane);
    if (POST) {
        loadj_async<J>(yq, a.post_y + 4 * lane);
        loadj_async<J>(pq, a.post_w + 4 * lane);
    }
    const int ngroups_mine =
        a.ngroups > (int)blockIdx.x ? (a.ngroups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
    const int nk = ngroups_mine * G;   // rows this wave copies
#pragma unroll
    for (int b = 0; b < NB - 1; ++b)
        if (b < nk) issue(b, b);
    wait_prologue<NB - 1, CI>(nk);
    pinj<J>(xq);
    if (a.norm) pinj<J>(nq);
    if (POST) {
        pinj<J>(yq);
        pinj<J>(pq);
    }
    float v[4 * J];   // v[4j + e] = x[256 j + 4 lane + e]
#pragma unroll
    for (int j = 0; j < J; ++j) {
        v[4 * j] = xq[j].x;
        v[4 * j + 1] = xq[j].y;
        v[4 * j + 2] = xq[j].z;
        v[4 * j + 3] = xq[j].w;
    }
    // x := x + post_w * (r_y * post_y) (rmsnorm_add_kernel's arithmetic); the
    // first workgroup stores it
    if (POST) {
        float sy = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            sy += yq[j].x * yq[j].x;
            sy += yq[j].y * yq[j].y;
            sy += yq[j].z * yq[j].z;
            sy += yq[j].w * yq[j].w;
        }
        sy = wave_sum(sy);
        const float ry = 1.0f / sqrtf(sy * a.inv_n + a.eps);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            v[4 * j] = v[4 * j] + pq[j].x * (ry * yq[j].x);
            v[4 * j + 1] = v[4 * j + 1] + pq[j].y * (ry * yq[j].y);
            v[4 * j + 2] = v[4 * j + 2] + pq[j].z * (ry * yq[j].z);
            v[4 * j + 3] = v[4 * j + 3] + pq[j].w * (ry * yq[j].w);
        }
        if (blockIdx.x == 0) {
#pragma unroll
            for (int j = 0; j < J; ++j)
                *reinterpret_cast<float4*>(a.post_out + 256 * j + 4 * lane) =
                    make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
        }
    }
    // RMSNorm: the lanes take w[i] * x[i], and the row totals are scaled by
    // r (the GEMV is linear in x)
    float rscale = 1.0f;
    if (a.norm) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 4 * J; ++i) ss += v[i] * v[i];
        ss = wave_sum(ss);
        rscale = 1.0f / sqrtf(ss * a.inv_n + a.eps);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            v[4 * j] = nq[j].x * v[4 * j];
            v[4 * j + 1] = nq[j].y * v[4 * j + 1];
            v[4 * j + 2] = nq[j].z * v[4 * j + 2];
            v[4 * j + 3] = nq[j].w * v[4 * j + 3];
        }
    }
    // lane geometry in a row buffer: the quant dword and byte shift, and the
    // scale's halfword, of group 0 (group j: + 68 j dwords, + 136 j halfwords)
    const uint32_t bl = (uint32_t)lane >> 3;
    const uint32_t qb = 34u * bl + 2u + 4u * ((uint32_t)lane & 7u);
    const uint32_t qdw = qb >> 2, sft = qb & 3u, sh = 17u * bl;

    for (int gl = 0; gl < ngroups_mine; ++gl) {
        float acc[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int k = gl * G + i;
            const int kn = k + NB - 1;
            if (kn < nk) issue(kn, kn % NB);
            wait_chunk<NB - 1, CI>(nk - 1 - k);
            const uint8_t* src;
            const bool real = chunk_src<G, PAIR>(cc, k, src);
            const uint32_t* buf = ring + (k % NB) * BDW;
            const uint16_t* hw = reinterpret_cast<const uint16_t*>(buf);
            float dv = 0.0f;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const uint32_t q = __builtin_amdgcn_alignbyte(buf[qdw + 68 * j + 1], buf[qdw + 68 * j], sft);
                const float d = h2f(hw[sh + 136 * j]);
                float s = (float)(int8_t)(q & 0xffu) * v[4 * j];
                s = fmaf((float)(int8_t)((q >> 8) & 0xffu), v[4 * j + 1], s);
                s = fmaf((float)(int8_t)((q >> 16) & 0xffu), v[4 * j + 2], s);
                s = fmaf((float)(int8_t)(q >> 24), v[4 * j + 3], s);
                dv = fmaf(s, d, dv);
            }
            asm volatile("" : "+v"(dv));
            acc[i] = real ? dv : 0.0f;
            wait_lgkm();   // this row's LDS reads are done before its buffer is refilled
        }
        float tot = xreduce<G>(acc, lane) * rscale;
        const int ri = rowof<G>(lane);
        const bool lead = (lane & ((64 / G) - 1)) == 0;
        const int grp = (int)blockIdx.x + gl * (int)gridDim.x;
        if constexpr (S > 1) {
            // the slices' row totals through LDS (two halves, so one barrier
            // per group suffices), added in slice order by the first wave
            float* red = xch + (gl & 1) * S * G;
            if (lead) red[sl * G + ri] = tot;
            lds_sync();
            if (sl != 0) continue;
            tot = red[ri];
#pragma unroll
            for (int q = 1; q < S; ++q) tot += red[q * G + ri];
        }
        if (PAIR) {
            if (lead) xch[ri] = tot;
            if (lane < NOUT) {
                const int row = grp * NOUT + lane;
                const float g = xch[lane], u = xch[lane + NOUT];
                if (row < a.rows[0]) a.y[0][row] = a.epilogue == EPI_GEGLU ? ref_geglu(g, u) : ref_swiglu(g, u);
            }
        } else if (lead) {
            const int gi = grp * G + ri;
            if (gi < a.rows_total) {
                int s, row;
                seg_of(a, gi, s, row);
                float* y = a.y[s] + row;
                if (a.epilogue == EPI_ADD) *y = *y + tot;
                else *y = tot;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------
int cus() { return device_cus(); }

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

template <int QT, int G, int NB, bool PAIR, bool UA>
int launch_rows(GemvArgs a, hipStream_t st) {
    constexpr int NOUT = PAIR ? G / 2 : G;
    const int nb = a.cols / 32;
    const int nw = (nb + 63) / 64;
    const int threads = nw * 64;
    const size_t base = (size_t)nw * NB * Fmt<QT>::kBufBytes + (size_t)2 * nw * G * 4 + (size_t)2 * nw * 4;
    auto lds_for = [&](int grid) { return base + (size_t)((a.ngroups + grid - 1) / grid) * NOUT * 4; };
    // the residual update is a separate instantiation: its registers would
    // otherwise count against every GEMV
    auto kern = a.post_y ? gemv_kernel<QT, G, NB, PAIR, UA, true> : gemv_kernel<QT, G, NB, PAIR, UA, false>;
    // Every workgroup reads the whole activation (and the norm weights when
    // fused), so workgroups per CU are also capped to keep that traffic near
    // 128 KB per CU: more workgroups than this only add x reads that compete
    // with the weight stream (measured on MI355X at the Llama-3-8B shapes).
    // The residual update's two vectors count too when the launch is short
    // (at most 4 row groups per workgroup at the plain cap), where they are a
    // large share of a workgroup's reads (Gemma-2-2B's q|k|v and gate|up);
    // long launches such as the LM head keep the plain cap.
    const int xbytes = a.cols * 4 * (a.norm ? 2 : 1);
    int xcap = std::max(1, (128 << 10) / xbytes);
    if (a.post_y && a.ngroups <= 4 * xcap * cus()) xcap = std::max(1, (128 << 10) / (xbytes + a.cols * 8));
    const int per_cu = std::min(occupancy(kern, threads, lds_for(cus())), xcap);
    const int cap = per_cu * cus();
    int grid = std::min(a.ngroups, cap);
    // Launches with the fused residual update keep the plain grid (cap
    // workgroups, one group more for the first ones): measured faster on
    // MI355X at Gemma-2-2B's q|k|v (9.56 -> 9.16 us) and LM head (117.1 ->
    // 112.9 us), while the balanced grid is faster for the others
    // (Llama-3-8B gate|up 24.9 -> 23.7 us).
    if (env_int("L3P_GEMV_BAL", 1) && !a.post_y) {
        // the same number of groups (k, or k-1 for the last few) per workgroup
        const int k = (a.ngroups + cap - 1) / cap;
        grid = (a.ngroups + k - 1) / k;
    }
    grid = std::max(grid, (a.ngroups * NOUT + kMaxOut - 1) / kMaxOut);
    // Row ranges when they take at least 20% of the rows off the busiest
    // CU.  The dispatcher places workgroup b on CU b mod CUs while every
    // workgroup of the launch is resident (breadth first), so a grid that is
    // not a multiple of the CUs loads some CUs with one workgroup more, and
    // the launch ends with them: Gemma-2-2B's 2304-row GEMVs in groups of 4
    // rows put 8 or 12 rows on a CU at 576 workgroups, 9 on every CU as 768
    // ranges of 3 rows (output projection 4.02 -> 3.70 us, down projection
    // 9.37 -> 8.76 us, measured on MI355X).  Small gains are left alone:
    // ranges spread the workgroups' streams over the whole matrix instead of
    // one band of it at a time, which made Gemma-2-2B's 590 MB LM head
    // slower (112 -> 122 us) for 0.6% fewer rows on its busiest CU; rows
    // dealt one by one over the workgroups kept the band but were no faster
    // at the small shapes (4.04 and 9.11 us).  At 12.5% (the 14336-row Q4_0
    // and Q4_K GEMVs: 64 -> 56 rows) ranges were 2-3% slower (p50 10.4-10.6
    // -> 10.7 us and 11.0-11.1 -> 11.2-11.4 us, alternating runs on one box).
    // Row ranges are built into the Q8_0 kernels without the residual update
    // (Gemma-2-2B's 2304-row output and down projections), where they gained.
    constexpr bool kRG = QT == L3P_Q8_0 && !PAIR;
    a.rpw = 0;
    size_t lds = lds_for(grid);
    if (kRG && !a.post_y && env_int("L3P_GEMV_RANGES", 1)) {
        const int n = cus();
        auto worst_cu = [&](int g, int rpw) {   // most rows on one CU
            std::vector<int> per(n, 0);
            for (int b = 0; b < g; ++b)
                per[b % n] += rpw ? std::max(0, std::min(rpw, a.rows_total - b * rpw))
                                  : (a.ngroups - b + g - 1) / g * G;
            return *std::max_element(per.begin(), per.end());
        };
        const int m = (grid + n - 1) / n;   // <= the workgroups per CU that fit (grid <= their count)
        const int rpw = (a.rows_total + m * n - 1) / (m * n);
        const int grid_r = (a.rows_total + rpw - 1) / rpw;
        const size_t lds_r = base + (size_t)((rpw + G - 1) / G) * G * 4;
        if ((rpw + G - 1) / G * G <= kMaxOut && lds_r <= lds_for(cus()) &&
            5 * worst_cu(grid_r, rpw) <= 4 * worst_cu(grid, 0)) {
            a.rpw = rpw;
            grid = grid_r;
            lds = lds_r;
        }
    }
    if constexpr (kRG) {
        if (a.rpw > 0) kern = gemv_kernel<QT, G, NB, PAIR, UA, false, true>;
    }
    if (lds > 65536)
        L3P_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    if (grid > kMaxSsParts) a.xw = nullptr;   // too many partial sums: the next GEMV takes its norm itself
    launch_kernel(kern, dim3(grid), dim3(threads), (uint32_t)lds, st, a);
    return a.xw ? grid : 0;
}

// Ring depth: 3 buffers per wave, 4 and 5 for Q8_0 and Q6_K launches with
// few waves per CU (see launch_type); 4 for chunks of at most 1280 bytes; 2
// for the 4 KB F16/BF16 and 8 KB F32 chunks of rows too wide for 3.
template <int QT, int G, bool PAIR, bool UA>
int launch_nb(GemvArgs a, int nbuf, hipStream_t st) {
    if constexpr (Fmt<QT>::kBufBytes >= 4096) {
        if (nbuf == 2) return launch_rows<QT, G, 2, PAIR, UA>(a, st);
    }
    if constexpr (Fmt<QT>::kChunkBytes <= 1280 || QT == L3P_Q8_0 || QT == L3P_Q6_K) {
        if (nbuf == 4) return launch_rows<QT, G, 4, PAIR, UA>(a, st);
    }
    if constexpr (QT == L3P_Q8_0 || QT == L3P_Q6_K) {
        if (nbuf == 5) return launch_rows<QT, G, 5, PAIR, UA>(a, st);
    }
    return launch_rows<QT, G, 3, PAIR, UA>(a, st);
}

template <int QT, bool UA>
int launch_g(GemvArgs a, bool pair, int G, int nbuf, hipStream_t st) {
    if (pair) {   // G counts gate and up rows together: 2 or 4 output rows per group
        switch (G) {
        case 4: return launch_nb<QT, 4, true, UA>(a, nbuf, st);
        default: return launch_nb<QT, 8, true, UA>(a, nbuf, st);
        }
    }
    switch (G) {
    case 4: return launch_nb<QT, 4, false, UA>(a, nbuf, st);
    case 16: return launch_nb<QT, 16, false, UA>(a, nbuf, st);
    default: return launch_nb<QT, 8, false, UA>(a, nbuf, st);
    }
}

// Whole-row launches (gemv_wide_kernel): one wave per workgroup, at most
// eight per CU, the same number of row groups per workgroup.
template <int J, int G, int NB, bool PAIR>
int launch_wide_rows(GemvArgs a, int wpc, hipStream_t st) {
    auto kern = a.post_y ? gemv_wide_kernel<J, G, NB, PAIR, true> : gemv_wide_kernel<J, G, NB, PAIR, false>;
    const size_t lds = (size_t)NB * wide_ci<J>() * 1024 + (size_t)G * 4;
    const int cap = std::min(occupancy(kern, 64, lds), wpc) * cus();
    const int k = (a.ngroups + cap - 1) / cap;
    const int grid = (a.ngroups + k - 1) / k;
    launch_kernel(kern, dim3(grid), dim3(64), (uint32_t)lds, st, a);
    return 0;
}
template <int J, int G, bool PAIR>
int launch_wide_nb(GemvArgs a, int wpc, int nb, hipStream_t st) {
    switch (nb) {
    case 3: return launch_wide_rows<J, G, 3, PAIR>(a, wpc, st);
    case 5: return launch_wide_rows<J, G, 5, PAIR>(a, wpc, st);
    default: return launch_wide_rows<J, G, 4, PAIR>(a, wpc, st);
    }
}
template <int J>
int launch_wide_g(GemvArgs a, bool pair, int G, int wpc, int nb, hipStream_t st) {
    if (pair) return G == 4 ? launch_wide_nb<J, 4, true>(a, wpc, nb, st) : launch_wide_nb<J, 8, true>(a, wpc, nb, st);
    switch (G) {
    case 2: return launch_wide_nb<J, 2, false>(a, wpc, nb, st);
    case 4: return launch_wide_nb<J, 4, false>(a, wpc, nb, st);
    case 16: return launch_wide_nb<J, 16, false>(a, wpc, nb, st);
    default: return launch_wide_nb<J, 8, false>(a, wpc, nb, st);
    }
}
// Four rows per group (two gate and two up rows for a pair) and up to eight
// waves per CU, measured on MI355X at Gemma-2-2B's 2304 columns (rocprof
// medians in the decode step, with the residual update fused): gate|up
// 12.9-13.1 us at six and eight waves per CU (14.6 at four, 13.8 at ten;
// 13.2 with eight rows per group at ten), q|k|v 5.7 us (6.7 and 6.9 with two
// and eight rows per group), the 256000-row LM head 102 us at eight (145,
// 123, 107 and 105 at four, six, ten and twelve), against 17.8, 9.0 and
// 115 us for the chunk-column kernel; ring depths 3 and 5 were slower than 4.
int launch_wide(GemvArgs a, bool pair, hipStream_t st) {
    const int units = pair ? a.rows[0] : a.rows_total;
    int wpc = env_int("L3P_GEMV_WIDE_WPC", 0);
    if (wpc <= 0) wpc = 8;
    int G = env_int("L3P_GEMV_WIDE_G", 0);
    if (G != 2 && G != 4 && G != 8 && G != 16) G = 4;
    if (pair && G == 16) G = 8;
    if (pair && G == 2) G = 4;
    const int per = pair ? G / 2 : G;
    a.ngroups = (units + per - 1) / per;
    const int nb = env_int("L3P_GEMV_WIDE_NB", 4);
    if (a.cols == 2304) return launch_wide_g<9>(a, pair, G, wpc, nb, st);
    return launch_wide_g<10>(a, pair, G, wpc, nb, st);
}

// Rows of S x 2304 columns: a workgroup of S waves takes one row at a time,
// each wave a 2304-column slice through its own 4-deep ring (the whole-row
// kernel's lane layout), and the first wave adds the slices' totals.  Rows
// are dealt evenly over as many workgroups as fit at once (Gemma-2-2B's 2304
// x 9216 down projection: 768 workgroups of three rows, three per CU).
template <int S>
int launch_sliced(GemvArgs a, hipStream_t st) {
    constexpr int J = 9, G = 1, NB = 4;
    auto kern = gemv_wide_kernel<J, G, NB, false, false, S>;
    const size_t lds = (size_t)S * NB * wide_ci<J>() * 1024 + (size_t)2 * S * G * 4;
    a.ngroups = a.rows_total;
    const int cap = std::max(1, occupancy(kern, 64 * S, lds)) * cus();
    const int k = (a.ngroups + cap - 1) / cap;
    const int grid = (a.ngroups + k - 1) / k;
    launch_kernel(kern, dim3(grid), dim3(64 * S), (uint32_t)lds, st, a);
    return 0;
}

template <int QT>
int launch_type(GemvArgs a, bool pair, int G, bool standalone, hipStream_t st) {
    const int units = pair ? a.rows[0] : a.rows_total;
    const int per = pair ? G / 2 : G;
    a.ngroups = (units + per - 1) / per;
    // three buffers per wave when they fit the 160 KB of LDS with room for
    // the result slots, else two (gemv_supported keeps F32 rows narrow enough)
    const int nw = (a.cols / 32 + 63) / 64;
    int nb = (size_t)nw * 3 * Fmt<QT>::kBufBytes + 16384 <= 160 * 1024 ? 3 : 2;
    // chunks of at most 1280 bytes (Q4_0, Q4_1, IQ4_NL, Q2_K, Q3_K, Q4_K) keep
    // three in flight: 5-6% faster at the Q4_0 and Q4_K FFN shapes, where
    // a 2-deep ring leaves too few bytes in flight per CU (measured on MI355X)
    if (Fmt<QT>::kChunkBytes <= 1280) nb = 4;
    // A CU's stream runs at the bytes it has in flight over the ~0.6 us load
    // latency, up to about 40 GB/s a CU (measured on MI355X): standalone Q8_0
    // and Q6_K launches with few waves per CU (the 4096 x 4096 Q8_0 GEMV: 4
    // waves a CU, two 2176-byte chunks each in flight) take a deeper ring,
    // until about 28 KB per CU are in flight (4096 x 4096: 7.64 -> 6.85 us
    // mean).  Inside the decode step the same rings were slower (the output
    // projection 6.92 -> 7.36 us, q|k|v 8.08 -> 8.20 us), so it keeps three.
    // The waves count the row's chunk columns as fractions (a 256-column
    // last column is an eighth of a chunk).
    if constexpr (QT == L3P_Q8_0 || QT == L3P_Q6_K) {
        const double kb = standalone ? env_int("L3P_GEMV_INFLIGHT_KB", 28) : 0;
        const double wpc = (double)std::min(a.ngroups, 4 * cus()) * a.cols / kChunkElems / cus();
        while (nb < 5 && wpc * (nb - 1) * Fmt<QT>::kChunkBytes < kb * 1024 &&
               (size_t)nw * (nb + 1) * Fmt<QT>::kBufBytes + 16384 <= 160 * 1024)
            ++nb;
    }
    if (row_bytes<QT>(a.cols) % 16 == 0) return launch_g<QT, false>(a, pair, G, nb, st);
    // Q4_K, Q5_K, F16, BF16 and F32 rows are always 16-byte multiples
    if constexpr (!Fmt<QT>::kAligned) return launch_g<QT, true>(a, pair, G, nb, st);
    return 0;
}

}  // namespace

int device_cus() {
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

bool gemv_supported(int type, int cols) {
    int unit;
    switch (type) {
    case L3P_Q8_0: case L3P_Q4_0: case L3P_Q4_1: case L3P_Q5_0: case L3P_Q5_1: case L3P_IQ4_NL:
    case L3P_F16: case L3P_BF16: unit = 32; break;
    case L3P_Q2_K: case L3P_Q3_K: case L3P_Q4_K: case L3P_Q5_K: case L3P_Q6_K: unit = 256; break;
    case L3P_F32: return cols > 0 && cols % 32 == 0 && cols <= 16384;   // 8 KB chunks: two per wave fit LDS
    default: return false;
    }
    return cols > 0 && cols % unit == 0 && cols <= kMaxWaves * kChunkElems;
}

bool gemv_fp32_activation(int type) {
    switch (type) {
    case L3P_Q4_0: return !q8_act<L3P_Q4_0>();
    case L3P_Q4_1: return !q8_act<L3P_Q4_1>();
    case L3P_Q5_0: return !q8_act<L3P_Q5_0>();
    case L3P_Q5_1: return !q8_act<L3P_Q5_1>();
    case L3P_IQ4_NL: return !q8_act<L3P_IQ4_NL>();
    default: return true;
    }
}

int launch_gemv(int type, const GemvBatch& b, int cols, const float* x, const float* norm, float eps,
                hipStream_t st) {
    L3P_REQUIRE(gemv_supported(type, cols), L3P_E_UNSUPPORTED, "gemv: type %d with %d columns not supported",
                type, cols);
    L3P_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)norm & 15) == 0, L3P_E_INVALID,
                "gemv: activation and norm weights must be 16-byte aligned");
    GemvArgs a{};
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
    if (a.rows_total == 0) return 0;
    a.x = x;
    a.norm = norm;
    a.eps = eps;
    a.inv_n = 1.0f / (float)cols;
    a.post_y = b.post_y;
    a.post_w = b.post_w;
    a.post_out = b.post_out;
    L3P_REQUIRE(!b.post_y || (b.post_w && b.post_out && b.post_out != x && ((uintptr_t)b.post_y & 15) == 0 &&
                              ((uintptr_t)b.post_w & 15) == 0 && ((uintptr_t)b.post_out & 15) == 0),
                L3P_E_INVALID, "gemv: bad residual update arguments");
    // the residual-update kernels hold four activation vectors in registers
    // and are built for at most 512 threads (8 chunk waves)
    L3P_REQUIRE(!b.post_y || cols <= kMaxPostCols, L3P_E_UNSUPPORTED, "gemv: residual update over %d columns", cols);
    L3P_REQUIRE(!b.xw || (b.epilogue == EPI_ADD && b.nseg == 1 && !b.pair && b.xw_w && b.ssp), L3P_E_INVALID,
                "gemv: normed residual output needs one residual-add segment");
    L3P_REQUIRE(!b.ss || (!norm && gemv_fp32_activation(type) && ((uintptr_t)b.ss & 15) == 0), L3P_E_INVALID,
                "gemv: summed-square input needs fp32 activations and no norm");
    L3P_REQUIRE(!(b.ss || b.xw) || (!b.post_y && !b.pair), L3P_E_INVALID,
                "gemv: the normed residual hand-over takes one-segment launches without a residual update");
    a.xw = b.xw;
    a.xw_w = b.xw_w;
    a.ssp = b.ssp;
    a.ss = b.ss;
    a.ss_loads = (b.n_ss + 255) / 256;
    a.n_ss = b.n_ss;
    L3P_REQUIRE(!b.ss || (b.n_ss > 0 && b.n_ss <= kMaxSsParts), L3P_E_INVALID, "gemv: %d sums of squares", b.n_ss);
    // Q8_0 rows of 2304 or 2560 columns stream whole rows per wave; rows of
    // 4 x 2304 columns (Gemma-2-2B's down projection) four 2304-column slices
    // per workgroup
    if (type == L3P_Q8_0 && wide_cols(cols) && !b.xw && !b.ss && env_int("L3P_GEMV_WIDE", 1))
        return launch_wide(a, b.pair != 0, st);
    if (type == L3P_Q8_0 && (cols == 2 * 2304 || cols == 3 * 2304 || cols == 4 * 2304) && !b.pair && !b.post_y &&
        !norm && !b.xw && !b.ss && env_int("L3P_GEMV_SLICED", 1)) {
        if (cols == 2 * 2304) return launch_sliced<2>(a, st);
        if (cols == 3 * 2304) return launch_sliced<3>(a, st);
        return launch_sliced<4>(a, st);
    }
    // Rows per group G: the largest of 16, 8, 4 that still gives about six
    // waves per CU (groups x column chunks); ring depth 3.  (Measured on
    // MI355X at the Llama-3-8B shapes.)
    const int nw = (cols / 32 + 63) / 64;
    const int units = a.rows_total;
    const int per_g = b.pair ? 2 : 1;   // pair groups hold G/2 rows of each matrix
    auto waves = [&](int g) { return (long)(units * per_g + g - 1) / g * nw; };
    int G = env_int("L3P_GEMV_G", 0);
    if (b.pair && G == 16) G = 8;   // pair kernels exist for G = 4, 8
    if (G != 4 && G != 8 && G != 16) {
        G = 4;
        for (int g : {16, 8})
            if ((!b.pair || g <= 8) && waves(g) >= 6L * cus()) {
                G = g;
                break;
            }
        // rows of at most two chunk columns keep 8 rows per group down to
        // four waves per CU (Llama-3-8B wo, 4096 x 4096: 7.56 -> 7.24 us),
        // except with the residual update (Gemma-2-2B's 4096 x 2304 q|k|v:
        // 9.20 us at 4 rows, 9.24 at 8)
        if (G == 4 && nw <= 2 && !a.post_y && waves(8) >= 4L * cus()) G = 8;
    }
    const bool pr = b.pair != 0;
    const bool sa = b.standalone != 0;
    switch (type) {
    case L3P_Q8_0: return launch_type<L3P_Q8_0>(a, pr, G, sa, st);
    case L3P_Q4_0: return launch_type<L3P_Q4_0>(a, pr, G, sa, st);
    case L3P_Q4_1: return launch_type<L3P_Q4_1>(a, pr, G, sa, st);
    case L3P_Q5_0: return launch_type<L3P_Q5_0>(a, pr, G, sa, st);
    case L3P_Q5_1: return launch_type<L3P_Q5_1>(a, pr, G, sa, st);
    case L3P_IQ4_NL: return launch_type<L3P_IQ4_NL>(a, pr, G, sa, st);
    case L3P_Q2_K: return launch_type<L3P_Q2_K>(a, pr, G, sa, st);
    case L3P_Q3_K: return launch_type<L3P_Q3_K>(a, pr, G, sa, st);
    case L3P_Q4_K: return launch_type<L3P_Q4_K>(a, pr, G, sa, st);
    case L3P_Q5_K: return launch_type<L3P_Q5_K>(a, pr, G, sa, st);
    case L3P_Q6_K: return launch_type<L3P_Q6_K>(a, pr, G, sa, st);
    case L3P_F16: return launch_type<L3P_F16>(a, pr, G, sa, st);
    case L3P_F32: return launch_type<L3P_F32>(a, pr, G, sa, st);
    default: return launch_type<L3P_BF16>(a, pr, G, sa, st);
    }
}
