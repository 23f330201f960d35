// blocks.hip — GGUF block conversion kernels (gfx950): Q8_0 quantization of
// fp32 values (quantize_row_q8_0, llama3pure-c-engine.c:1508-1528), bit-exact
// dequantization of every supported type (dequantize_row_*, c:611-934) and
// the embedding-row gather of a decode step.
#include <algorithm>

#include "dequant.h"
#include "device_common.h"
#include "internal.h"

namespace {

using namespace l3pd;

// Q8_0 quantization of nb blocks of 32 values into GGUF block_q8_0 bytes.
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

__global__ void dequant_kernel(int type, const uint8_t* __restrict__ s, int64_t n, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = deq_elem(type, s, i);
}

// Embedding row (c:3204-3207), times a scale when non-zero (Gemma's sqrt(dim),
// which the reference applies to x in place before the first norm,
// c:3132-3140; x*scale rounds the same), the step record {token, pos} that
// the kernels of the step read, and the RoPE table rows of pos (when
// rope.rope_cur is set), so that attention need not wait for the record to
// find them.
__global__ void embed_step_kernel(int type, const uint8_t* __restrict__ s, int n, float scale, float* __restrict__ y,
                                  int token, int pos, int* step, RopeRows rope, const int* dtok, size_t rb,
                                  HostToken ht) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (dtok) {   // the token the previous step's sampler left on the device; s is row 0
        token = *dtok;
        s += (size_t)token * rb;
    } else if (ht.word) {   // the token the host's sampler finish hands over; s is row 0
        __shared__ int tok_s;
        if (threadIdx.x == 0) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            uint64_t w = __hip_atomic_load(ht.word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
            while ((uint32_t)(w >> 32) != ht.seq) {
                if (__builtin_amdgcn_s_memrealtime() - t0 > kHostWaitTicks) {   // the host never answered
                    __hip_atomic_store(ht.fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    w = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
                w = __hip_atomic_load(ht.word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            int t = (int)(uint32_t)w;
            if (t < 0 || t >= ht.vocab) {
                __hip_atomic_store(ht.fail, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                t = 0;
            }
            tok_s = t;
        }
        __syncthreads();
        token = tok_s;
        s += (size_t)token * rb;
    }
    if (i < n) {
        const float v = deq_elem(type, s, i);
        y[i] = scale != 0.0f ? v * scale : v;
    }
    if (i == 0) {
        step[0] = token;
        step[1] = pos;
    }
    if (rope.rope_cur && i < 4 * rope.half) {
        const int t = i / rope.half, j = i - t * rope.half;
        rope.rope_cur[i] = rope.tables[t][(size_t)pos * rope.half + j];
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A plain streaming read of n 16-byte words, the bandwidth ceiling the decode
// GEMVs' weight stream is compared with: each workgroup reads contiguous
// blocks of 256 x kSR words (eight nontemporal loads in flight per thread),
// folded into one value that is stored only in a case the data would have to
// be built for (which keeps the loads).
constexpr int kSR = 8;
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ p, size_t n, uint32_t* out) {
    const size_t stride = (size_t)gridDim.x * 256 * kSR;
    size_t i = (size_t)blockIdx.x * 256 * kSR + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (kSR - 1) * 256 < n; i += stride) {
        u32x4 v[kSR];
#pragma unroll
        for (int u = 0; u < kSR; ++u) v[u] = __builtin_nontemporal_load(p + i + u * 256);
#pragma unroll
        for (int u = 0; u < kSR; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (size_t j = i; j < n && j < i + kSR * 256; j += 256) {   // the one partial block
        const u32x4 v = __builtin_nontemporal_load(p + j);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) out[blockIdx.x & 255] = acc;
}

}  // namespace

void launch_stream_read(const void* p, size_t bytes, uint32_t* out, hipStream_t st) {
    const size_t n = bytes / 16;
    if (n == 0) return;
    const size_t want = (size_t)device_cus() * 8;   // 8 workgroups of 256 per CU
    const unsigned grid = (unsigned)std::min(want, (n + 256 * kSR - 1) / (256 * kSR));
    launch_kernel(stream_read_kernel, dim3(grid), dim3(256), 0u, st, reinterpret_cast<const u32x4*>(p), n, out);
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
                      const RopeRows* rope, hipStream_t st, const int* dtok, size_t rb, HostToken ht) {
    RopeRows r{};
    if (rope) r = *rope;
    const int threads = std::max(n, r.rope_cur ? 4 * r.half : 0);
    hipLaunchKernelGGL(embed_step_kernel, dim3((threads + 255) / 256), dim3(256), 0, st, type, row, n, scale, dst,
                       token, pos, step, r, dtok, rb, ht);
    L3P_HIP(hipGetLastError());
}
