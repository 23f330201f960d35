// dequant.h — bit-exact dequantization of one element of a GGUF tensor
// (dequantize_row_*, llama3pure-c-engine.c:611-934), shared by the
// dequantization, embedding and GEMM kernels.
#pragma once

#include "device_common.h"
#include "l3p.h"

namespace l3pd {

// ---------------------------------------------------------------------------
// Dequantization, one element per thread, bit-exact with dequantize_row
// (c:611-934) for the types listed in l3p.h.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float ldh(const uint8_t* p) { return h2f_exact((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

__device__ __forceinline__ float deq_elem(int type, const uint8_t* __restrict__ s, int64_t i) {
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
    case L3P_Q2_K: {   // dequantize_row_q2_K (c:748-784): group g = e / 16
        const uint8_t* b = s + (i >> 8) * 84;
        const int e = (int)(i & 255), g = e >> 4, l = e & 15;
        const int half = g >> 3, j = (g >> 1) & 3, second = g & 1;
        const int u = (b[16 + 32 * half + 16 * second + l] >> (2 * j)) & 3;
        const float dl = ldh(b + 80) * (float)(b[g] & 0x0f), ml = ldh(b + 82) * (float)(b[g] >> 4);
        return dl * (float)u - ml;
    }
    case L3P_Q3_K: {   // dequantize_row_q3_K (c:786-832)
        const uint8_t* b = s + (i >> 8) * 110;
        const int e = (int)(i & 255), g = e >> 4, l = e & 15;
        const int half = g >> 3, j = (g >> 1) & 3, second = g & 1;
        const uint8_t* sb = b + 96;
        const int lo = g < 8 ? (sb[g] & 0x0f) : (sb[g - 8] >> 4);
        const int sg = (lo | (((sb[8 + (g & 3)] >> (2 * (g >> 2))) & 3) << 4)) - 32;
        const int u = (b[32 + 32 * half + 16 * second + l] >> (2 * j)) & 3;
        const int h = (b[16 * second + l] >> (4 * half + j)) & 1;
        return (ldh(b + 108) * (float)sg) * (float)(u - (h ? 0 : 4));
    }
    case L3P_Q5_K: {   // dequantize_row_q5_K (c:834-871): sub-block k = e / 32
        const uint8_t* b = s + (i >> 8) * 176;
        const int e = (int)(i & 255), k = e >> 5, l = e & 31;
        const uint8_t* sc = b + 4;
        int scv, mnv;
        if (k < 4) {
            scv = sc[k] & 63;
            mnv = sc[k + 4] & 63;
        } else {
            scv = (sc[k + 4] & 0x0f) | ((sc[k - 4] >> 6) << 4);
            mnv = (sc[k + 4] >> 4) | ((sc[k] >> 6) << 4);
        }
        const uint8_t byte = b[48 + 32 * (k >> 1) + l];
        const int q = ((k & 1) ? (byte >> 4) : (byte & 0x0f)) + (((b[16 + l] >> k) & 1) ? 16 : 0);
        return (ldh(b) * (float)scv) * (float)q - ldh(b + 2) * (float)mnv;
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

}  // namespace l3pd
