// blocks.hip — GGUF block conversion kernels (gfx950): Q8_0 quantization of
// fp32 values (quantize_row_q8_0, llama3pure-c-engine.c:1508-1528), bit-exact
// dequantization of every supported type (dequantize_row_*, c:611-934) and
// the embedding-row gather of a decode step.
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

}  // namespace

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
