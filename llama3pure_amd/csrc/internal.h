// internal.h — shared declarations of libl3p (host and device).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <string>
#include <vector>

#include "../../include/l3p.h"

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
struct L3pError {
    int code;
    std::string msg;
};

#define L3P_HIP(expr)                                                                        \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess)                                                                \
            throw L3pError{L3P_E_HIP, std::string(#expr ": ") + hipGetErrorString(e_)};      \
    } while (0)

#define L3P_REQUIRE(cond, code, ...)                                                         \
    do {                                                                                     \
        if (!(cond)) {                                                                       \
            char b_[512];                                                                    \
            snprintf(b_, sizeof b_, __VA_ARGS__);                                            \
            throw L3pError{code, b_};                                                        \
        }                                                                                    \
    } while (0)

// ---------------------------------------------------------------------------
// kernel timing: a timed range (ProfRange) hands an event pair to the next
// GEMV or GEMM launch, which has the dispatch itself record them at the
// kernel's start and end (hipExtLaunchKernelGGL), so the range measures the
// kernel alone and not the stream's dispatch latency around it.
// ---------------------------------------------------------------------------
struct KernelEvents {
    hipEvent_t start = nullptr, stop = nullptr;   // null: no range open
    int launches = 0;                             // launches inside the open range
};
KernelEvents& kernel_events();   // per host thread

template <typename K, typename... Args>
void launch_kernel(K kern, dim3 grid, dim3 block, uint32_t lds, hipStream_t st, Args... args) {
    KernelEvents& ke = kernel_events();
    if (ke.start && ke.launches++ == 0)
        hipExtLaunchKernelGGL(kern, grid, block, lds, st, ke.start, ke.stop, 0, args...);
    else
        hipLaunchKernelGGL(kern, grid, block, lds, st, args...);
    L3P_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// block formats (llama3pure-c-engine.c:127-195)
// ---------------------------------------------------------------------------
inline int type_block_elems(int t) {
    switch (t) {
    case L3P_Q4_0: case L3P_Q4_1: case L3P_Q5_0: case L3P_Q5_1: case L3P_Q8_0: case L3P_IQ4_NL:
        return 32;
    case L3P_Q2_K: case L3P_Q3_K: case L3P_Q4_K: case L3P_Q5_K: case L3P_Q6_K:
        return 256;
    case L3P_F32: case L3P_F16: case L3P_BF16:
        return 1;
    default:
        return 0;
    }
}
inline int type_block_bytes(int t) {
    switch (t) {
    case L3P_F32: return 4;
    case L3P_F16: case L3P_BF16: return 2;
    case L3P_Q4_0: return 18;
    case L3P_Q4_1: return 20;
    case L3P_Q5_0: return 22;
    case L3P_Q5_1: return 24;
    case L3P_Q8_0: return 34;
    case L3P_Q2_K: return 84;
    case L3P_Q3_K: return 110;
    case L3P_Q4_K: return 144;
    case L3P_Q5_K: return 176;
    case L3P_Q6_K: return 210;
    case L3P_IQ4_NL: return 18;
    default: return 0;
    }
}
inline size_t type_row_bytes(int t, int64_t cols) {
    int e = type_block_elems(t);
    return e ? (size_t)(cols / e) * (size_t)type_block_bytes(t) : 0;
}

// ---------------------------------------------------------------------------
// GEMV launch descriptions
// ---------------------------------------------------------------------------
enum GemvEpilogue : int {
    EPI_STORE = 0,   // y[r] = W.x
    EPI_ADD = 1,     // y[r] += W.x          (residual add, c:3111-3115)
    EPI_SWIGLU = 2,  // pair (gate, up): y[r] = silu(g) * u      (c:3400-3406)
    EPI_GEGLU = 3,   // pair (gate, up): y[r] = gelu_tanh(g) * u  (c:3391-3398)
};

// Up to three matrices sharing one input vector, run in one launch
// (q/k/v, or gate/up with a fused activation).
struct GemvSegment {
    const uint8_t* w;
    float* y;
    int rows;
};
struct GemvBatch {
    GemvSegment seg[3];
    int nseg;
    int pair;      // 1: seg[0] and seg[1] are (gate, up) processed together
    int epilogue;  // GemvEpilogue
    // 1: a launch on its own (l3p_gemv), not inside a decode step: Q8_0 and
    // Q6_K rows then take a copy ring deep enough for the launch's waves per
    // CU (measured faster there, slower inside the decode step)
    int standalone;
    // Optional residual update before the GEMV's own norm (Gemma's post
    // norms): x := x + post_w * rmsnorm(post_y) with the GEMV's eps and width,
    // the updated x written to post_out (not x: the launch's workgroups all
    // read x) by the first workgroup.
    const float* post_y;
    const float* post_w;
    float* post_out;
    // Optional, for a residual add (EPI_ADD, one segment): every output i
    // also goes to xw[i] as y[i] * xw_w[i] (the next RMSNorm's weights), and
    // ssp[g] receives workgroup g's sum of y[i]^2 over its outputs, in a
    // fixed order; ssp holds kMaxSsParts floats, and entries past this
    // launch's grid keep whatever an earlier, larger grid wrote (consumers
    // read only the first n_ss).
    float* xw;
    const float* xw_w;
    float* ssp;
    // Optional, for a GEMV whose weights take fp32 activations: x is already
    // the residual times the norm weights (norm null), and its RMSNorm's sum
    // of squares is the sum of the n_ss floats at ss (n_ss <= kMaxSsParts).
    const float* ss;
    int n_ss;
};
// Widest rows a GEMV with the residual update takes (8 column chunks).
constexpr int kMaxPostCols = 16384;
// Workgroups of a residual-add GEMV whose sums of squares a later GEMV reads.
constexpr int kMaxSsParts = 1024;

// gemv.hip: the decode GEMV over Q8_0 / Q4_0 / Q4_K / Q6_K rows, with an
// optional RMSNorm of x fused into its prologue (norm != null).  Weights, x
// and norm must be 16-byte aligned.
bool gemv_supported(int type, int cols);
// whether the type's GEMV takes the activation in fp32 (not as Q8_0 blocks)
bool gemv_fp32_activation(int type);
// returns the number of partial sums of squares written to b.ssp (0 without
// b.xw, or when the launch has more than kMaxSsParts workgroups: then xw and
// ssp are not written)
int launch_gemv(int type, const GemvBatch& b, int cols, const float* x, const float* norm, float eps,
                hipStream_t s);
// gemm.hip: Y[m][n] (=|+=) W[n,:] . X[m,:] on the fp32 matrix cores, for the
// types the reference dequantizes before its batched dot (Q8_0, the K-quants,
// F16, BF16, F32).  x rows must be 16-byte aligned (ldx a multiple of 4).
// One launch takes up to three matrices of one type and K over the same X
// (q|k|v, gate|up); with a workspace ws of ws_floats floats, K is split when
// the output tiles are too few to fill the GPU.
struct GemmSegment {
    const uint8_t* w;
    int n;        // output features (weight rows)
    float* y;
    int ldy;
};
struct GemmJob {
    int type;
    GemmSegment seg[3];
    int nseg;
    int k;
    const float* x;
    int m, ldx;
    bool add;
};
bool gemm_mfma_supported(int type);
// the types whose batched dot takes Q8_0-quantized activation rows (Q4_0,
// Q4_1, Q5_0, Q5_1, IQ4_NL): the int8 matrix-core path, exact block dots
bool gemm_q8_activation(int type);
// workspace floats the int8 path needs for `rows` activation rows of k columns
size_t gemm_q8a_ws_floats(int rows, int k);
// the job through workspace ws (the rows in as many launches as it needs)
void launch_gemm_q8a(const GemmJob& j, float* ws, size_t ws_floats, hipStream_t s);
void launch_gemm(const GemmJob& j, float* ws, size_t ws_floats, hipStream_t s);
// K splits of a job and the fp32 partials they need, for a workspace of
// ws_floats floats (0: no split)
struct GemmPlan {
    int nsplit = 1, ksteps = 0;   // stream-K: nsplit = most partial slots of a tile, ksteps = K steps of a tile
    int bn = 64;   // output columns per tile: 64, or 128 when those tiles fill the CUs unsplit
    int streamk = 0;   // > 0: stream-K over that many workgroups
    size_t partial_floats = 0;
};
GemmPlan gemm_plan(const GemmJob& j, size_t ws_floats);
void launch_gemm_planned(const GemmJob& j, const GemmPlan& plan, float* ws, hipStream_t s);
// split-K partials of a context (allocated with it): 64 MB
constexpr size_t kGemmWsFloats = (size_t)16 << 20;
// the file-scope partials array of l3p_gemm_static (16 MB per GPU) and its
// device address on the current device
constexpr size_t kGemmStaticScratchFloats = (size_t)4 << 20;
float* gemm_static_scratch();
// compute units of the current device
int device_cus();
// blocks.hip
void launch_quantize_q8_0_blocks(const float* x, int64_t n, uint8_t* dst, hipStream_t s);
void launch_dequant(int type, const uint8_t* src, int64_t n, float* dst, hipStream_t s);
// a plain streaming read of bytes (a multiple of 16) from 16-byte aligned p;
// out: 256 words of device scratch
void launch_stream_read(const void* p, size_t bytes, uint32_t* out, hipStream_t s);
// rope (may be null): copies the four RoPE table rows of pos (tables[t] +
// pos * half, t = 0..3) into rope_cur[t * half ..]
struct RopeRows {
    const float* tables[4];
    int half;
    float* rope_cur;
};
// A token handed over by the host through coherent pinned memory: the step
// waits until *word holds (seq << 32) | token (word null: no such wait).  The
// wait is bounded (kHostWaitTicks of the 100 MHz realtime counter): past it,
// or for a token outside [0, vocab), the step runs with token 0 and sets
// *fail, which the host reports.
struct HostToken {
    const uint64_t* word;
    uint32_t seq;
    uint32_t* fail;
    int vocab;
};
constexpr uint64_t kHostWaitTicks = 1000000000ull;   // 10 s
// dtok: read the token from device memory instead (row is then row 0 and
// rb the row stride in bytes); ht.word: wait for it from the host (likewise)
void launch_embed_row(int type, const uint8_t* row, int n, float scale, float* dst, int token, int pos, int* step,
                      const RopeRows* rope, hipStream_t s, const int* dtok = nullptr, size_t rb = 0,
                      HostToken ht = HostToken{});
// Top-k slots published to coherent pinned host memory by the scan kernel:
// the k values and indices, then *seq_word = seq once they are visible
// (v null: not published).
struct HostSlots {
    float* v;
    int* i;
    uint32_t* seq_word;
    uint32_t seq;
};
