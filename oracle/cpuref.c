/*
 * cpuref.c — CPU restatement (the oracle) of llama3pure's quantized forward
 * path.  TEST INFRASTRUCTURE ONLY: the product (libl3p.so, HIP) never links or
 * calls this file; tests/, smoke() and bench.py's cpu_baseline use it as the
 * checker.
 *
 * Each function names the reference lines (llama3pure-c-engine.c, "c:LINE")
 * whose arithmetic it restates.  The order of every fp32 operation is kept, and
 * the file is compiled with -ffp-contract=off so no multiply-add is fused,
 * exactly like the reference's `gcc -O3` build on x86-64 (Makefile:7-8), which
 * has no FMA instructions to contract into.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   - fp16 table: exhaustive against IEEE binary16 (numpy) and oracle/_ref.
 *   - truncating fp32->fp16: edge classes + 2^20 random floats vs oracle/_ref.
 *   - dequantizers: exact-rational closed forms + golden fixtures from _ref.
 *   - Q8_0 quantizer: closed form (amax/127, roundf) + ties + _ref fixtures.
 *   - matmul: bit-identical to _ref's matmul_quantized; float64 bound.
 *   - forward/prefill: bit-identical logits and KV bytes vs _ref on synthetic
 *     GGUF models (Llama and Gemma arch).
 *   - sampler: xorshift64* KAT + brute-force restatement vs _ref generate_token.
 */
#include "cpuref.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define QK8 32
#define QKK 256
#define Q8_BYTES 34

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32                                                             */
/* ------------------------------------------------------------------------ */

static float g_half_table[65536];
static int g_half_ready = 0;

static float bits_to_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f32_to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* c:547-582: normalises subnormals by shifting the mantissa until bit 10 is
 * set; exponent 31 keeps the NaN payload in the float mantissa. */
static void half_table_init(void) {
    if (g_half_ready) return;
    for (uint32_t h = 0; h < 65536; h++) {
        uint32_t sign = (h & 0x8000u) << 16;
        int32_t e = (int32_t)((h >> 10) & 0x1f);
        uint32_t m = h & 0x3ffu;
        uint32_t out;
        if (e == 0 && m == 0) {
            out = sign;
        } else if (e == 31) {
            out = sign | 0x7f800000u | (m << 13);
        } else {
            if (e == 0) {              /* subnormal: renormalise */
                while (!(m & 0x400u)) { m <<= 1; e--; }
                e++;
                m &= 0x3ffu;
            }
            out = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
        }
        g_half_table[h] = bits_to_f32(out);
    }
    g_half_ready = 1;
}

float l3o_fp16_to_fp32(uint16_t h) { half_table_init(); return g_half_table[h]; }

/* c:585-599: mantissa truncated (no rounding); exponents below the subnormal
 * range flush to signed zero; overflow (and NaN) become signed infinity. */
uint16_t l3o_fp32_to_fp16(float f) {
    uint32_t b = f32_to_bits(f);
    uint32_t sign = (b >> 16) & 0x8000u;
    int e = (int)((b >> 23) & 0xffu) - 112;
    uint32_t m = (b >> 13) & 0x3ffu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        return (uint16_t)(sign | ((m | 0x400u) >> (1 - e)));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | m);
}

void l3o_fp16_to_fp32_n(const uint16_t* h, float* f, size_t n) {
    half_table_init();
    for (size_t i = 0; i < n; i++) f[i] = g_half_table[h[i]];
}
void l3o_fp32_to_fp16_n(const float* f, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; i++) h[i] = l3o_fp32_to_fp16(f[i]);
}

static inline float h2f(const uint8_t* p) { return g_half_table[(uint16_t)(p[0] | (p[1] << 8))]; }

/* ------------------------------------------------------------------------ */
/* block formats (c:127-206, c:1049-1091)                                    */
/* ------------------------------------------------------------------------ */

int l3o_block_elems(int type) {
    switch (type) {
    case L3O_Q4_0: case L3O_Q4_1: case L3O_Q5_0: case L3O_Q5_1: case L3O_Q8_0: case L3O_IQ4_NL:
        return 32;
    case L3O_Q2_K: case L3O_Q3_K: case L3O_Q4_K: case L3O_Q5_K: case L3O_Q6_K:
        return 256;
    default:
        return 1;
    }
}

size_t l3o_block_bytes(int type) {
    switch (type) {
    case L3O_F32: return 4;
    case L3O_F16: case L3O_BF16: case L3O_BF16_ALT: return 2;
    case L3O_Q4_0: return 18;
    case L3O_Q4_1: return 20;
    case L3O_Q5_0: return 22;
    case L3O_Q5_1: return 24;
    case L3O_Q8_0: return 34;
    case L3O_Q2_K: return 84;
    case L3O_Q3_K: return 110;
    case L3O_Q4_K: return 144;
    case L3O_Q5_K: return 176;
    case L3O_Q6_K: return 210;
    case L3O_IQ4_NL: return 18;
    default: return 0;
    }
}

size_t l3o_row_bytes(int type, int cols) {
    return (size_t)(cols / l3o_block_elems(type)) * l3o_block_bytes(type);
}

/* ------------------------------------------------------------------------ */
/* dequantizers                                                              */
/* ------------------------------------------------------------------------ */

static void dq_q8_0(const uint8_t* s, float* y, int n) {          /* c:691-702 */
    for (int b = 0; b < n / 32; b++, s += 34) {
        float d = h2f(s);
        const int8_t* q = (const int8_t*)(s + 2);
        for (int j = 0; j < 32; j++) y[32 * b + j] = q[j] * d;
    }
}

static void dq_q4_0(const uint8_t* s, float* y, int n) {          /* c:611-626 */
    for (int b = 0; b < n / 32; b++, s += 18) {
        float d = h2f(s);
        for (int j = 0; j < 16; j++) {
            y[32 * b + j] = ((s[2 + j] & 0x0f) - 8) * d;
            y[32 * b + j + 16] = ((s[2 + j] >> 4) - 8) * d;
        }
    }
}

static void dq_q4_1(const uint8_t* s, float* y, int n) {          /* c:628-645 */
    for (int b = 0; b < n / 32; b++, s += 20) {
        float d = h2f(s), m = h2f(s + 2);
        for (int j = 0; j < 16; j++) {
            y[32 * b + j] = (s[4 + j] & 0x0f) * d + m;
            y[32 * b + j + 16] = (s[4 + j] >> 4) * d + m;
        }
    }
}

static void dq_q5_0(const uint8_t* s, float* y, int n) {          /* c:647-668 */
    for (int b = 0; b < n / 32; b++, s += 22) {
        float d = h2f(s);
        uint32_t qh = (uint32_t)s[2] | ((uint32_t)s[3] << 8) | ((uint32_t)s[4] << 16) | ((uint32_t)s[5] << 24);
        for (int j = 0; j < 16; j++) {
            int lo = (s[6 + j] & 0x0f) | (int)(((qh >> j) & 1u) << 4);
            int hi = (s[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
            y[32 * b + j] = (lo - 16) * d;
            y[32 * b + j + 16] = (hi - 16) * d;
        }
    }
}

static void dq_q5_1(const uint8_t* s, float* y, int n) {          /* c:670-689 */
    for (int b = 0; b < n / 32; b++, s += 24) {
        float d = h2f(s), m = h2f(s + 2);
        uint32_t qh = (uint32_t)s[4] | ((uint32_t)s[5] << 8) | ((uint32_t)s[6] << 16) | ((uint32_t)s[7] << 24);
        for (int j = 0; j < 16; j++) {
            int lo = (s[8 + j] & 0x0f) | (int)(((qh >> j) & 1u) << 4);
            int hi = (s[8 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
            y[32 * b + j] = lo * d + m;
            y[32 * b + j + 16] = hi * d + m;
        }
    }
}

/* c:705-714: 6-bit scale/min unpacking for Q4_K/Q5_K. */
static void k4_scale_min(int j, const uint8_t* q, int* sc, int* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

static void dq_q4_k(const uint8_t* s, float* y, int n) {          /* c:716-746 */
    for (int b = 0; b < n / 256; b++, s += 144) {
        float d = h2f(s), dmin = h2f(s + 2);
        const uint8_t* sc = s + 4;
        const uint8_t* q = s + 16;
        for (int g = 0; g < 4; g++) {           /* 64 elements per group */
            int s0, m0, s1, m1;
            k4_scale_min(2 * g, sc, &s0, &m0);
            k4_scale_min(2 * g + 1, sc, &s1, &m1);
            float d0 = d * s0, mm0 = dmin * m0, d1 = d * s1, mm1 = dmin * m1;
            for (int l = 0; l < 32; l++) y[256 * b + 64 * g + l] = d0 * (q[32 * g + l] & 0x0f) - mm0;
            for (int l = 0; l < 32; l++) y[256 * b + 64 * g + 32 + l] = d1 * (q[32 * g + l] >> 4) - mm1;
        }
    }
}

static void dq_q6_k(const uint8_t* s, float* y, int n) {          /* c:873-904 */
    for (int b = 0; b < n / 256; b++, s += 210) {
        const uint8_t* ql = s;
        const uint8_t* qh = s + 128;
        const int8_t* sc = (const int8_t*)(s + 192);
        float d = h2f(s + 208);
        for (int half = 0; half < 2; half++) {
            float* o = y + 256 * b + 128 * half;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[l] = d * sc[is + 0] * q1;
                o[l + 32] = d * sc[is + 2] * q2;
                o[l + 64] = d * sc[is + 4] * q3;
                o[l + 96] = d * sc[is + 6] * q4;
            }
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* Q2_K super-block {u8 scales[16]; u8 qs[64]; fp16 d, dmin} (c:165-170):
 * 16 groups of 16 elements; group g has scale byte scales[g] (low nibble the
 * scale, high nibble the min) and 2-bit codes from qs[32*(g/8) + 16*(g%2) + l]
 * at bit shift 2*((g/2)%4).  y = (d*sc)*u - (dmin*m)  (c:748-784). */
static void dq_q2_k(const uint8_t* s, float* y, int n) {
    for (int b = 0; b < n / 256; b++, s += 84) {
        const uint8_t* sc = s;
        const uint8_t* qs = s + 16;
        float d = h2f(s + 80), dmin = h2f(s + 82);
        for (int g = 0; g < 16; g++) {
            int half = g / 8, shift = 2 * ((g / 2) % 4), second = g % 2;
            float dl = d * (float)(sc[g] & 0x0f), ml = dmin * (float)(sc[g] >> 4);
            for (int l = 0; l < 16; l++) {
                int u = (qs[32 * half + 16 * second + l] >> shift) & 3;
                y[256 * b + 16 * g + l] = dl * (float)u - ml;
            }
        }
    }
}

/* The 16 six-bit scales of a Q3_K super-block from its 12 packed bytes
 * (c:802-806): scale i has its low 4 bits in byte i (low nibble) for i < 8
 * or byte i - 8 (high nibble) for i >= 8, and its high 2 bits in byte
 * 8 + i%4 at bit 2*(i/4). */
static int q3k_scale(const uint8_t* p, int i) {
    int lo = i < 8 ? (p[i] & 0x0f) : (p[i - 8] >> 4);
    int hi = (p[8 + (i % 4)] >> (2 * (i / 4))) & 3;
    return lo | (hi << 4);
}

/* Q3_K super-block {u8 hmask[32]; u8 qs[64]; u8 scales[12]; fp16 d}
 * (c:172-178): group g of 16 elements uses qs and the shift as in Q2_K, the
 * high bit hmask[16*(g%2) + l] bit (4*(g/8) + (g/2)%4), value
 * u - (bit ? 0 : 4), scale d*(s_g - 32)  (c:786-832). */
static void dq_q3_k(const uint8_t* s, float* y, int n) {
    for (int b = 0; b < n / 256; b++, s += 110) {
        const uint8_t* hm = s;
        const uint8_t* qs = s + 32;
        const uint8_t* scp = s + 96;
        float d = h2f(s + 108);
        for (int g = 0; g < 16; g++) {
            int half = g / 8, j = (g / 2) % 4, second = g % 2;
            float dl = d * (float)(q3k_scale(scp, g) - 32);
            int bit = 4 * half + j;
            for (int l = 0; l < 16; l++) {
                int u = (qs[32 * half + 16 * second + l] >> (2 * j)) & 3;
                int h = (hm[16 * second + l] >> bit) & 1;
                y[256 * b + 16 * g + l] = dl * (float)(u - (h ? 0 : 4));
            }
        }
    }
}

/* Q5_K super-block {fp16 d, dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]}
 * (c:180-187): sub-block k (32 elements) is the low (k even) or high nibble
 * of qs[32*(k/2) + l] plus 16 * bit k of qh[l], with the Q4_K 6-bit scale and
 * min k: y = (d*sc)*q - (dmin*m)  (c:834-871). */
static void dq_q5_k(const uint8_t* s, float* y, int n) {
    for (int b = 0; b < n / 256; b++, s += 176) {
        float d = h2f(s), dmin = h2f(s + 2);
        const uint8_t* sc = s + 4;
        const uint8_t* qh = s + 16;
        const uint8_t* qs = s + 48;
        for (int k = 0; k < 8; k++) {
            int scv, mnv;
            k4_scale_min(k, sc, &scv, &mnv);
            float dk = d * (float)scv, mk = dmin * (float)mnv;
            for (int l = 0; l < 32; l++) {
                int nib = (k & 1) ? (qs[32 * (k / 2) + l] >> 4) : (qs[32 * (k / 2) + l] & 0x0f);
                int q = nib + (((qh[l] >> k) & 1) ? 16 : 0);
                y[256 * b + 32 * k + l] = dk * (float)q - mk;
            }
        }
    }
}

static const int8_t k_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                   1,    13,   25,  38,  53,  69,  89,  113};   /* c:204-206 */

static void dq_iq4_nl(const uint8_t* s, float* y, int n) {        /* c:922-934 */
    for (int b = 0; b < n / 32; b++, s += 18) {
        float d = h2f(s);
        for (int j = 0; j < 16; j++) {
            y[32 * b + j] = d * k_iq4nl[s[2 + j] & 0x0f];
            y[32 * b + j + 16] = d * k_iq4nl[s[2 + j] >> 4];
        }
    }
}

int l3o_dequant_row(int type, const void* src, float* dst, int n) {   /* c:1003-1046 */
    const uint8_t* s = (const uint8_t*)src;
    half_table_init();
    switch (type) {
    case L3O_F32: memcpy(dst, src, (size_t)n * 4); return 0;
    case L3O_F16: for (int i = 0; i < n; i++) dst[i] = h2f(s + 2 * i); return 0;
    case L3O_BF16: case L3O_BF16_ALT:
        for (int i = 0; i < n; i++) dst[i] = bits_to_f32((uint32_t)(s[2 * i] | (s[2 * i + 1] << 8)) << 16);
        return 0;
    case L3O_Q4_0: dq_q4_0(s, dst, n); return 0;
    case L3O_Q4_1: dq_q4_1(s, dst, n); return 0;
    case L3O_Q5_0: dq_q5_0(s, dst, n); return 0;
    case L3O_Q5_1: dq_q5_1(s, dst, n); return 0;
    case L3O_Q8_0: dq_q8_0(s, dst, n); return 0;
    case L3O_Q2_K: dq_q2_k(s, dst, n); return 0;
    case L3O_Q3_K: dq_q3_k(s, dst, n); return 0;
    case L3O_Q4_K: dq_q4_k(s, dst, n); return 0;
    case L3O_Q5_K: dq_q5_k(s, dst, n); return 0;
    case L3O_Q6_K: dq_q6_k(s, dst, n); return 0;
    case L3O_IQ4_NL: dq_iq4_nl(s, dst, n); return 0;
    default: return -1;
    }
}

/* c:1508-1528 (and the identical KV-cache variant c:1535-1570): per block of
 * 32, d = amax/127, id = 127/amax (not 1/d), q = roundf(x*id) clamped. */
void l3o_quantize_q8_0(const float* x, void* dst, int n) {
    uint8_t* o = (uint8_t*)dst;
    for (int b = 0; b < n / 32; b++, o += 34) {
        const float* xb = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = xb[j] < 0 ? -xb[j] : xb[j];
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d > 0.0f ? 127.0f / amax : 0.0f;
        uint16_t h = l3o_fp32_to_fp16(d);
        o[0] = (uint8_t)(h & 0xff);
        o[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) {
            int q = (int)roundf(xb[j] * id);
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            ((int8_t*)(o + 2))[j] = (int8_t)q;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV                                                                      */
/* ------------------------------------------------------------------------ */

static int has_row_dequant(int type) {   /* get_deq_row_func, c:2063-2073 */
    return type == L3O_Q8_0 || type == L3O_Q2_K || type == L3O_Q3_K || type == L3O_Q4_K ||
           type == L3O_Q5_K || type == L3O_Q6_K;
}

/* Integer dot of a Q8_0 activation against one Q4_0 row (c:1625-1643). */
static float dot_q4_0_q8_0(const uint8_t* xq, const uint8_t* w, int n) {
    float sum = 0.0f;
    for (int b = 0; b < n / 32; b++, w += 18, xq += 34) {
        float dw = h2f(w), dx = h2f(xq);
        const int8_t* xs = (const int8_t*)(xq + 2);
        int isum = 0;
        for (int j = 0; j < 16; j++) {
            isum += xs[j] * ((w[2 + j] & 0x0f) - 8) + xs[j + 16] * ((w[2 + j] >> 4) - 8);
        }
        sum += dw * dx * (float)isum;
    }
    return sum;
}

/* Q8_0 activation against one Q4_1 row (c:1646-1665): per block the exact
 * integer dots isum = sum xq*u and xsum = sum xq, then
 * sum += dw*dx*isum + mw*dx*xsum. */
static float dot_q4_1_q8_0(const uint8_t* xq, const uint8_t* w, int n) {
    float sum = 0.0f;
    for (int b = 0; b < n / 32; b++, w += 20, xq += 34) {
        float dw = h2f(w), mw = h2f(w + 2), dx = h2f(xq);
        const int8_t* xs = (const int8_t*)(xq + 2);
        int isum = 0, xsum = 0;
        for (int j = 0; j < 16; j++) {
            isum += xs[j] * (w[4 + j] & 0x0f) + xs[j + 16] * (w[4 + j] >> 4);
            xsum += xs[j] + xs[j + 16];
        }
        sum += dw * dx * (float)isum + mw * dx * (float)xsum;
    }
    return sum;
}

/* The 5-bit code of element j (< 32) of a Q5_0 / Q5_1 block: nibble of
 * qs[j % 16] (low for j < 16) and bit j of the 32-bit qh. */
static int q5_code(const uint8_t* qh4, const uint8_t* qs, int j) {
    uint32_t qh = (uint32_t)qh4[0] | ((uint32_t)qh4[1] << 8) | ((uint32_t)qh4[2] << 16) | ((uint32_t)qh4[3] << 24);
    int nib = j < 16 ? (qs[j] & 0x0f) : (qs[j - 16] >> 4);
    return nib | (int)(((qh >> j) & 1u) << 4);
}

/* Q8_0 activation against one Q5_0 row (c:1668-1690): isum = sum xq*(u-16),
 * sum += dw*dx*isum. */
static float dot_q5_0_q8_0(const uint8_t* xq, const uint8_t* w, int n) {
    float sum = 0.0f;
    for (int b = 0; b < n / 32; b++, w += 22, xq += 34) {
        float dw = h2f(w), dx = h2f(xq);
        const int8_t* xs = (const int8_t*)(xq + 2);
        int isum = 0;
        for (int j = 0; j < 32; j++) isum += xs[j] * (q5_code(w + 2, w + 6, j) - 16);
        sum += dw * dx * (float)isum;
    }
    return sum;
}

/* Q8_0 activation against one Q5_1 row (c:1693-1717): isum = sum xq*u,
 * xsum = sum xq, sum += dw*dx*isum + mw*dx*xsum. */
static float dot_q5_1_q8_0(const uint8_t* xq, const uint8_t* w, int n) {
    float sum = 0.0f;
    for (int b = 0; b < n / 32; b++, w += 24, xq += 34) {
        float dw = h2f(w), mw = h2f(w + 2), dx = h2f(xq);
        const int8_t* xs = (const int8_t*)(xq + 2);
        int isum = 0, xsum = 0;
        for (int j = 0; j < 32; j++) {
            isum += xs[j] * q5_code(w + 4, w + 8, j);
            xsum += xs[j];
        }
        sum += dw * dx * (float)isum + mw * dx * (float)xsum;
    }
    return sum;
}

/* Q8_0 activation against one IQ4_NL row (c:1994-2011): the nibbles index
 * the 16-value table, isum = sum xq*table[u], sum += dw*dx*isum. */
static float dot_iq4_nl_q8_0(const uint8_t* xq, const uint8_t* w, int n) {
    float sum = 0.0f;
    for (int b = 0; b < n / 32; b++, w += 18, xq += 34) {
        float dw = h2f(w), dx = h2f(xq);
        const int8_t* xs = (const int8_t*)(xq + 2);
        int isum = 0;
        for (int j = 0; j < 16; j++)
            isum += xs[j] * k_iq4nl[w[2 + j] & 0x0f] + xs[j + 16] * k_iq4nl[w[2 + j] >> 4];
        sum += dw * dx * (float)isum;
    }
    return sum;
}

/* Integer dot of a Q8_0 activation against one Q8_0 row (c:1720-1736). */
static float dot_q8_0_q8_0(const uint8_t* xq, const uint8_t* w, int n) {
    float sum = 0.0f;
    for (int b = 0; b < n / 32; b++, w += 34, xq += 34) {
        float dw = h2f(w), dx = h2f(xq);
        const int8_t* xs = (const int8_t*)(xq + 2);
        const int8_t* ws = (const int8_t*)(w + 2);
        int isum = 0;
        for (int j = 0; j < 32; j++) isum += xs[j] * ws[j];
        sum += dw * dx * (float)isum;
    }
    return sum;
}

static int is_q8_act(int type) {   /* q8_func without a row dequantizer (c:2091-2133) */
    return type == L3O_Q4_0 || type == L3O_Q4_1 || type == L3O_Q5_0 || type == L3O_Q5_1 || type == L3O_IQ4_NL;
}

static int is_float_type(int type) {
    return type == L3O_F32 || type == L3O_F16 || type == L3O_BF16 || type == L3O_BF16_ALT;
}

/* Rows dequantized to fp32, then for each batch element b the sequential fp32
 * dot y[b][r] = sum_j w[r][j] * x[b][j], j = 0, 1, ... in order: the per-row
 * arithmetic of matmul_deq_4row / matmul_deq_batch_4row (c:2136-2273) and of
 * the float dots vec_dot_f16/bf16/f32 (c:1467-1494; x*w and w*x round alike).
 * Rows are taken kRowBlock at a time, each row its own accumulation chain, and
 * the blocks are spread over OpenMP threads, as the reference spreads its row
 * groups (c:2145, c:2189); no row's value depends on the thread count. */
enum { kRowBlock = 8 };
/* Eight fp32 lanes, one per row of a block: every operation on it is the
 * lane-wise IEEE multiply or add, so lane r accumulates exactly the sequence
 * s_r += w[r][j] * x[j] that a scalar loop over j would. */
typedef float v8f __attribute__((vector_size(32)));

static int deq_rows_dot(int type, const uint8_t* wb, size_t rb, int rows, int cols, const float* x, int batch,
                        int ldx, float* y, int ldy) {
    const int nblk = (rows + kRowBlock - 1) / kRowBlock;
    int err = 0;
#pragma omp parallel
    {
        /* the block's rows interleaved: wt[j] = {w[r0][j], .., w[r0 + 7][j]} */
        v8f* wt = (v8f*)aligned_alloc(32, (size_t)cols * sizeof(v8f));
        float* row = (float*)malloc((size_t)cols * sizeof(float));
        if (!wt || !row) {
#pragma omp atomic write
            err = 1;
        }
#pragma omp for schedule(static)
        for (int g = 0; g < nblk; g++) {
            if (!wt || !row) continue;
            const int r0 = g * kRowBlock;
            const int nr = rows - r0 < kRowBlock ? rows - r0 : kRowBlock;
            for (int r = 0; r < kRowBlock; r++) {
                if (r < nr) {
                    if (l3o_dequant_row(type, wb + (size_t)(r0 + r) * rb, row, cols) != 0) {
#pragma omp atomic write
                        err = 1;
                    }
                } else {
                    memset(row, 0, (size_t)cols * sizeof(float));
                }
                for (int j = 0; j < cols; j++) wt[j][r] = row[j];
            }
            int b = 0;
            for (; b + 1 < batch; b += 2) {   /* two independent chains per lane */
                const float* x0 = x + (size_t)b * ldx;
                const float* x1 = x0 + ldx;
                v8f s0 = {0}, s1 = {0};
                for (int j = 0; j < cols; j++) {
                    s0 = s0 + wt[j] * x0[j];
                    s1 = s1 + wt[j] * x1[j];
                }
                for (int r = 0; r < nr; r++) {
                    y[(size_t)b * ldy + r0 + r] = s0[r];
                    y[(size_t)(b + 1) * ldy + r0 + r] = s1[r];
                }
            }
            if (b < batch) {
                const float* x0 = x + (size_t)b * ldx;
                v8f s0 = {0};
                for (int j = 0; j < cols; j++) s0 = s0 + wt[j] * x0[j];
                for (int r = 0; r < nr; r++) y[(size_t)b * ldy + r0 + r] = s0[r];
            }
        }
        free(wt);
        free(row);
    }
    return err ? -1 : 0;
}

/* The Q8_0-activation types: each batch element quantized to Q8_0 once, then
 * the integer block dot of every row (c:2105-2116, c:2305-2318). */
static int q8_rows_dot(int type, const uint8_t* wb, size_t rb, int rows, int cols, const float* x, int batch,
                       int ldx, float* y, int ldy) {
    float (*dot)(const uint8_t*, const uint8_t*, int) =
        type == L3O_Q4_0 ? dot_q4_0_q8_0 : type == L3O_Q4_1 ? dot_q4_1_q8_0 :
        type == L3O_Q5_0 ? dot_q5_0_q8_0 : type == L3O_Q5_1 ? dot_q5_1_q8_0 : dot_iq4_nl_q8_0;
    const size_t qb = (size_t)(cols / 32) * 34;
    uint8_t* xq = (uint8_t*)malloc(qb * (size_t)(batch > 0 ? batch : 1));
    if (!xq) return -1;
    for (int b = 0; b < batch; b++) l3o_quantize_q8_0(x + (size_t)b * ldx, xq + (size_t)b * qb, cols);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < batch; b++) y[(size_t)b * ldy + r] = dot(xq + (size_t)b * qb, wb + (size_t)r * rb, cols);
    free(xq);
    return 0;
}

/* matmul_quantized (c:2091-2133): rows with a row dequantizer (Q8_0, Q2_K
 * .. Q6_K) go through matmul_deq_4row (c:2136-2176): dequantize to fp32 then
 * a sequential fp32 dot `s += w[j]*x[j]`.  Q4_0, Q4_1, Q5_0, Q5_1 and IQ4_NL
 * quantize x to Q8_0 once and use their integer block dots.  F32/F16/BF16
 * take the float dot (sequential, c:1467-1494). */
int l3o_matmul(int type, const void* w, int rows, int cols, const float* x, float* y) {
    return l3o_matmul_batch(type, w, rows, cols, x, 1, cols, y, rows);
}

/* matmul_quantized_batch (c:2291-2331) computes, for every batch element,
 * exactly what matmul_quantized computes for that element alone; here every
 * row is dequantized once for the whole batch, as matmul_deq_batch_4row
 * does (c:2179-2273). */
int l3o_matmul_batch(int type, const void* w, int rows, int cols, const float* x, int batch,
                     int in_stride, float* y, int out_stride) {
    const uint8_t* wb = (const uint8_t*)w;
    const size_t rb = l3o_row_bytes(type, cols);
    half_table_init();
    if (rows <= 0 || batch <= 0) return rows < 0 || batch < 0 ? -1 : 0;
    if (has_row_dequant(type) || is_float_type(type))
        return deq_rows_dot(type, wb, rb, rows, cols, x, batch, in_stride, y, out_stride);
    if (is_q8_act(type)) return q8_rows_dot(type, wb, rb, rows, cols, x, batch, in_stride, y, out_stride);
    return -1;
}

/* ------------------------------------------------------------------------ */
/* elementwise                                                               */
/* ------------------------------------------------------------------------ */

float l3o_fast_tanhf(float x) {                                   /* c:3089-3095 */
    if (x < -4.0f) return -1.0f;
    if (x > 4.0f) return 1.0f;
    float x2 = x * x;
    return (x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2)))) /
           (135135.0f + x2 * (62370.0f + x2 * (3150.0f + 28.0f * x2)));
}

float l3o_fast_expf(float x) {                                    /* c:3098-3106 */
    if (x > 10.0f) return 22026.47f;
    if (x < -10.0f) return 0.0f;
    float x2 = x * x;
    float x3 = x2 * x;
    float num = 120.0f + 60.0f * x + 12.0f * x2 + x3;
    float den = 120.0f - 60.0f * x + 12.0f * x2 - x3;
    return num / den;
}

/* c:3117-3129.  `inv` is 1.0f/(float)n as cached by malloc_run_state. */
static void rmsnorm_inv(float* o, const float* x, const float* w, int n, float inv, float eps) {
    float ss = 0.0f;
    for (int j = 0; j < n; j++) ss += x[j] * x[j];
    ss = 1.0f / sqrtf(ss * inv + eps);
    for (int j = 0; j < n; j++) o[j] = w[j] * (ss * x[j]);
}

void l3o_rmsnorm(float* o, const float* x, const float* w, int n, float eps) {
    rmsnorm_inv(o, x, w, n, 1.0f / (float)n, eps);
}

void l3o_softmax(float* x, int n) {                               /* c:3167-3186 */
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

void l3o_swiglu(float* hb, const float* hb2, int n) {             /* c:3400-3406 */
    for (int i = 0; i < n; i++) {
        float v = hb[i];
        v = v * (1.0f / (1.0f + l3o_fast_expf(-v)));
        hb[i] = v * hb2[i];
    }
}

void l3o_geglu(float* hb, const float* hb2, int n) {              /* c:3391-3398 */
    for (int i = 0; i < n; i++) {
        float x = hb[i];
        float g = 0.5f * x * (1.0f + l3o_fast_tanhf(x * (0.7978845608f + 0.035677408137f * x * x)));
        hb[i] = g * hb2[i];
    }
}

/* ------------------------------------------------------------------------ */
/* sampler                                                                   */
/* ------------------------------------------------------------------------ */

uint32_t l3o_rng_u32(uint64_t* s) {                               /* c:4266-4272 */
    *s ^= *s >> 12;
    *s ^= *s << 25;
    *s ^= *s >> 27;
    return (uint32_t)((*s * 0x2545F4914F6CDD1Dull) >> 32);
}

float l3o_rng_f32(uint64_t* s) { return (l3o_rng_u32(s) >> 8) / 16777216.0f; }   /* c:4274-4276 */

int l3o_argmax(const float* v, int n) {                           /* c:4278-4288 */
    int bi = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++) if (v[i] > bv) { bi = i; bv = v[i]; }
    return bi;
}

/* The sampling branch of generate_token (c:4803-4907): top-k by
 * min-replacement, temperature softmax over k, insertion sort, top-p cut,
 * one xorshift64* draw. */
int l3o_sample(const float* logits, int n, float temperature, int top_k, float top_p, uint64_t* rng) {
    if (temperature == 0.0f) return l3o_argmax(logits, n);
    int k = top_k > n ? n : top_k;
    int* idx = (int*)malloc((size_t)k * sizeof(int));
    float* val = (float*)malloc((size_t)k * sizeof(float));
    for (int i = 0; i < k; i++) { idx[i] = i; val[i] = logits[i]; }
    int mpos = 0;
    float mval = val[0];
    for (int i = 1; i < k; i++) if (val[i] < mval) { mval = val[i]; mpos = i; }
    for (int i = k; i < n; i++) {
        if (logits[i] > mval) {
            val[mpos] = logits[i];
            idx[mpos] = i;
            mval = val[0];
            mpos = 0;
            for (int j = 1; j < k; j++) if (val[j] < mval) { mval = val[j]; mpos = j; }
        }
    }
    float it = 1.0f / temperature;
    float mx = val[0];
    for (int i = 1; i < k; i++) if (val[i] > mx) mx = val[i];
    float mxt = mx * it;
    float sum = 0.0f;
    for (int i = 0; i < k; i++) { float e = expf(val[i] * it - mxt); val[i] = e; sum += e; }
    int keep = k;
    if (top_p < 1.0f) {
        for (int i = 1; i < k; i++) {
            float kv = val[i];
            int ki = idx[i];
            int j = i - 1;
            while (j >= 0 && val[j] < kv) { val[j + 1] = val[j]; idx[j + 1] = idx[j]; j--; }
            val[j + 1] = kv;
            idx[j + 1] = ki;
        }
        float cum = 0.0f, thr = top_p * sum;
        keep = k;
        for (int i = 0; i < k; i++) {
            cum += val[i];
            if (cum >= thr) { keep = i + 1; break; }
        }
        sum = 0.0f;
        for (int i = 0; i < keep; i++) sum += val[i];
    }
    float r = l3o_rng_f32(rng) * sum;
    float cdf = 0.0f;
    int s = keep - 1;
    for (int i = 0; i < keep; i++) {
        cdf += val[i];
        if (r < cdf) { s = i; break; }
    }
    int tok = idx[s];
    free(idx);
    free(val);
    return tok;
}

/* ------------------------------------------------------------------------ */
/* GGUF (in memory) and model                                                */
/* ------------------------------------------------------------------------ */

static char g_err[512];
const char* l3o_last_error(void) { return g_err; }
#define FAIL(...) do { snprintf(g_err, sizeof g_err, __VA_ARGS__); goto fail; } while (0)

typedef struct { const char* key; size_t klen; uint32_t type; const uint8_t* val; uint64_t alen; uint32_t atype; } kv_t;
typedef struct { const char* name; size_t nlen; uint32_t ndim; uint64_t ne[4]; uint32_t type; uint64_t off; } ti_t;
typedef struct { const uint8_t* data; int type; int rows, cols; size_t rb; } qt_t;

struct l3o_model {
    /* config (c:201-219) */
    int dim, hidden, n_layers, n_heads, n_kv, vocab, seq_len, head_dim, is_gemma;
    float theta, theta_swa, eps, softcap;
    int swa_window, swa_pattern;
    float attn_softcap;   /* load option, no counterpart in the reference: 0 = off */
    /* weights (c:251-278) */
    qt_t emb;
    float *att_norm, *ffn_norm, *final_norm, *q_norm, *k_norm, *post_att_norm, *post_ffn_norm;
    qt_t *wq, *wk, *wv, *wo, *w1, *w2, *w3, wcls;
    /* run state (c:281-343) */
    int hs, kv_dim, q_dim, max_dim, kv_mul, hq8;
    size_t head_seq, layer_kv;
    float attn_scale, embed_scale, inv_dim, inv_hs;
    float *x, *xb, *xb2, *hb, *hb2, *q, *k, *v, *att, *logits;
    uint8_t *kc, *vc, *qq8, *xq8;
    float *cos_d, *sin_d, *cos_s, *sin_s;
};

typedef struct { const uint8_t* p; const uint8_t* end; int bad; } rd_t;
static uint64_t rd_u(rd_t* r, int n) {
    uint64_t v = 0;
    if (r->p + n > r->end) { r->bad = 1; return 0; }
    for (int i = 0; i < n; i++) v |= (uint64_t)r->p[i] << (8 * i);
    r->p += n;
    return v;
}
static int type_size(uint32_t t) {
    static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return t < 13 ? sz[t] : -1;
}
static void rd_skip_value(rd_t* r, uint32_t t) {
    if (t == 8) { uint64_t n = rd_u(r, 8); if ((uint64_t)(r->end - r->p) < n) r->bad = 1; else r->p += n; return; }
    if (t == 9) {
        uint32_t at = (uint32_t)rd_u(r, 4);
        uint64_t n = rd_u(r, 8);
        for (uint64_t i = 0; i < n && !r->bad; i++) rd_skip_value(r, at);
        return;
    }
    int s = type_size(t);
    if (s <= 0) { r->bad = 1; return; }
    if (r->p + s > r->end) r->bad = 1; else r->p += s;
}

static const kv_t* find_kv(const kv_t* kv, uint64_t n, const char* key) {
    size_t kl = strlen(key);
    for (uint64_t i = 0; i < n; i++) if (kv[i].klen == kl && !memcmp(kv[i].key, key, kl)) return &kv[i];
    return NULL;
}
static int64_t kv_int(const kv_t* kv, uint64_t n, const char* key, int64_t dflt) {   /* c:2447-2463 */
    const kv_t* e = find_kv(kv, n, key);
    if (!e) return dflt;
    const uint8_t* v = e->val;
    switch (e->type) {
    case 0: return v[0];
    case 1: return (int8_t)v[0];
    case 2: return (uint16_t)(v[0] | v[1] << 8);
    case 3: return (int16_t)(v[0] | v[1] << 8);
    case 4: { uint32_t u; memcpy(&u, v, 4); return u; }
    case 5: { int32_t u; memcpy(&u, v, 4); return u; }
    case 10: { uint64_t u; memcpy(&u, v, 8); return (int64_t)u; }
    case 11: { int64_t u; memcpy(&u, v, 8); return u; }
    default: return dflt;
    }
}
static float kv_float(const kv_t* kv, uint64_t n, const char* key, float dflt) {     /* c:2466-2475 */
    const kv_t* e = find_kv(kv, n, key);
    if (!e) return dflt;
    if (e->type == 6) { float f; memcpy(&f, e->val, 4); return f; }
    if (e->type == 12) { double d; memcpy(&d, e->val, 8); return (float)d; }
    return dflt;
}
static int kv_str_eq(const kv_t* kv, uint64_t n, const char* key, const char* s) {
    const kv_t* e = find_kv(kv, n, key);
    if (!e || e->type != 8) return 0;
    uint64_t len; memcpy(&len, e->val, 8);
    return len == strlen(s) && !memcmp(e->val + 8, s, len);
}

static const ti_t* find_t(const ti_t* t, uint64_t n, const char* name) {
    size_t nl = strlen(name);
    for (uint64_t i = 0; i < n; i++) if (t[i].nlen == nl && !memcmp(t[i].name, name, nl)) return &t[i];
    return NULL;
}

static float* load_float(const ti_t* t, const uint8_t* base, int n) {   /* c:2838-2869 */
    float* o = (float*)malloc((size_t)n * sizeof(float));
    if (!o) return NULL;
    if (l3o_dequant_row((int)t->type, base + t->off, o, n) != 0) { free(o); return NULL; }
    return o;
}

l3o_model* l3o_model_open(const void* gguf, size_t len, int context_size) {
    half_table_init();
    l3o_model* m = (l3o_model*)calloc(1, sizeof(l3o_model));
    kv_t* kv = NULL;
    ti_t* ti = NULL;
    rd_t r = {(const uint8_t*)gguf, (const uint8_t*)gguf + len, 0};
    if (!m) FAIL("out of memory");
    if (rd_u(&r, 4) != 0x46554747u) FAIL("bad GGUF magic");                 /* c:2500-2531 */
    uint32_t ver = (uint32_t)rd_u(&r, 4);
    if (ver < 2 || ver > 3) FAIL("unsupported GGUF version %u", ver);
    uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
    if (r.bad || nt > (1u << 20) || nkv > (1u << 20)) FAIL("truncated GGUF header");
    kv = (kv_t*)calloc(nkv + 1, sizeof(kv_t));
    ti = (ti_t*)calloc(nt + 1, sizeof(ti_t));
    int64_t vocab_tokens = -1;
    for (uint64_t i = 0; i < nkv; i++) {
        uint64_t kl = rd_u(&r, 8);
        if (r.bad || (uint64_t)(r.end - r.p) < kl) FAIL("truncated GGUF metadata");
        kv[i].key = (const char*)r.p; kv[i].klen = kl; r.p += kl;
        kv[i].type = (uint32_t)rd_u(&r, 4);
        kv[i].val = r.p;
        if (kv[i].type == 9) {
            kv[i].atype = (uint32_t)rd_u(&r, 4);
            kv[i].alen = rd_u(&r, 8);
            r.p = kv[i].val;
            if (kl == 21 && !memcmp(kv[i].key, "tokenizer.ggml.tokens", 21) && kv[i].atype == 8)
                vocab_tokens = (int64_t)kv[i].alen;                          /* c:2717-2721 */
        }
        rd_skip_value(&r, kv[i].type);
        if (r.bad) FAIL("truncated GGUF metadata value");
    }
    for (uint64_t i = 0; i < nt; i++) {
        uint64_t nl = rd_u(&r, 8);
        if (r.bad || (uint64_t)(r.end - r.p) < nl) FAIL("truncated tensor info");
        ti[i].name = (const char*)r.p; ti[i].nlen = nl; r.p += nl;
        ti[i].ndim = (uint32_t)rd_u(&r, 4);
        if (ti[i].ndim > 4) FAIL("tensor with %u dims", ti[i].ndim);
        for (uint32_t d = 0; d < ti[i].ndim; d++) ti[i].ne[d] = rd_u(&r, 8);
        ti[i].type = (uint32_t)rd_u(&r, 4);
        ti[i].off = rd_u(&r, 8);
        if (r.bad) FAIL("truncated tensor info");
    }
    uint64_t align = (uint64_t)kv_int(kv, nkv, "general.alignment", 32);      /* c:2617-2621 */
    uint64_t hdr = (uint64_t)(r.p - (const uint8_t*)gguf);
    uint64_t data_off = (hdr + align - 1) / align * align;
    if (data_off > len) FAIL("truncated GGUF data");
    const uint8_t* base = (const uint8_t*)gguf + data_off;
    for (uint64_t i = 0; i < nt; i++) {
        uint64_t ne = 1;
        for (uint32_t d = 0; d < ti[i].ndim; d++) ne *= ti[i].ne[d];
        int be = l3o_block_elems((int)ti[i].type);
        size_t bb = l3o_block_bytes((int)ti[i].type);
        if (bb == 0) FAIL("unsupported tensor type %u", ti[i].type);
        if (data_off + ti[i].off + ne / be * bb > len) FAIL("tensor data out of file");
    }

    /* config, as main() builds it (c:5049-5145) */
    const char* pre = "llama";
    m->is_gemma = kv_str_eq(kv, nkv, "general.architecture", "gemma3") ||
                  kv_str_eq(kv, nkv, "general.architecture", "gemma2") ||
                  kv_str_eq(kv, nkv, "general.architecture", "gemma");
    if (m->is_gemma) {
        pre = "gemma3";
        if (kv_int(kv, nkv, "gemma3.embedding_length", 0) == 0) {
            if (kv_int(kv, nkv, "gemma2.embedding_length", 0) != 0) pre = "gemma2";
            else if (kv_int(kv, nkv, "gemma.embedding_length", 0) != 0) pre = "gemma";
        }
    }
    char key[96];
#define KEY(s) (snprintf(key, sizeof key, "%s." s, pre), key)
    m->swa_window = (int)kv_int(kv, nkv, KEY("attention.sliding_window"), 0);
    m->theta_swa = kv_float(kv, nkv, KEY("rope.freq_base_swa"), 10000.0f);
    m->swa_pattern = 6;
    m->dim = (int)kv_int(kv, nkv, KEY("embedding_length"), 4096);
    m->hidden = (int)kv_int(kv, nkv, KEY("feed_forward_length"), 11008);
    m->n_layers = (int)kv_int(kv, nkv, KEY("block_count"), 32);
    m->n_heads = (int)kv_int(kv, nkv, KEY("attention.head_count"), 32);
    m->n_kv = (int)kv_int(kv, nkv, KEY("attention.head_count_kv"), m->n_heads);
    m->vocab = (int)kv_int(kv, nkv, KEY("vocab_size"), 32000);
    m->seq_len = (int)kv_int(kv, nkv, KEY("context_length"), 2048);
    m->theta = kv_float(kv, nkv, KEY("rope.freq_base"), m->is_gemma ? 1000000.0f : 500000.0f);
    m->head_dim = (int)kv_int(kv, nkv, KEY("attention.key_length"), m->dim / m->n_heads);
    m->eps = kv_float(kv, nkv, KEY("attention.layer_norm_rms_epsilon"), 1e-6f);
    m->softcap = kv_float(kv, nkv, KEY("final_logit_softcapping"), 0.0f);
#undef KEY
    if (vocab_tokens > 0 && vocab_tokens != m->vocab) m->vocab = (int)vocab_tokens;   /* c:5152-5157 */
    if (context_size > 0 && context_size < m->seq_len) m->seq_len = context_size;        /* c:5174-5178 */
    if (m->head_dim % 32 || m->dim % 32 || m->n_kv <= 0 || m->n_heads % m->n_kv) FAIL("unsupported dims");

    int hs = m->head_dim;
    m->hs = hs;
    m->kv_dim = m->n_kv * hs;
    m->q_dim = m->n_heads * hs;
    m->max_dim = m->dim > m->q_dim ? m->dim : m->q_dim;
    m->kv_mul = m->n_heads / m->n_kv;

    /* weights (c:2939-3082) */
    const ti_t* t = find_t(ti, nt, "token_embd.weight");
    if (!t) FAIL("missing token_embd.weight");
    m->emb.data = base + t->off; m->emb.type = (int)t->type; m->emb.rows = m->vocab; m->emb.cols = m->dim;
    m->emb.rb = l3o_row_bytes(m->emb.type, m->dim);
    int L = m->n_layers;
    m->att_norm = (float*)malloc((size_t)L * m->dim * 4);
    m->ffn_norm = (float*)malloc((size_t)L * m->dim * 4);
    m->wq = (qt_t*)calloc(L, sizeof(qt_t)); m->wk = (qt_t*)calloc(L, sizeof(qt_t));
    m->wv = (qt_t*)calloc(L, sizeof(qt_t)); m->wo = (qt_t*)calloc(L, sizeof(qt_t));
    m->w1 = (qt_t*)calloc(L, sizeof(qt_t)); m->w2 = (qt_t*)calloc(L, sizeof(qt_t));
    m->w3 = (qt_t*)calloc(L, sizeof(qt_t));
    if (m->is_gemma) {
        m->q_norm = (float*)malloc((size_t)L * hs * 4); m->k_norm = (float*)malloc((size_t)L * hs * 4);
        m->post_att_norm = (float*)malloc((size_t)L * m->dim * 4);
        m->post_ffn_norm = (float*)malloc((size_t)L * m->dim * 4);
    }
    char nm[128];
    for (int l = 0; l < L; l++) {
        struct { const char* sfx; float* dst; int n; } fl[6] = {
            {"attn_norm.weight", m->att_norm + (size_t)l * m->dim, m->dim},
            {"ffn_norm.weight", m->ffn_norm + (size_t)l * m->dim, m->dim},
            {"attn_q_norm.weight", m->q_norm ? m->q_norm + (size_t)l * hs : NULL, hs},
            {"attn_k_norm.weight", m->k_norm ? m->k_norm + (size_t)l * hs : NULL, hs},
            {"post_attention_norm.weight", m->post_att_norm ? m->post_att_norm + (size_t)l * m->dim : NULL, m->dim},
            {"post_ffw_norm.weight", m->post_ffn_norm ? m->post_ffn_norm + (size_t)l * m->dim : NULL, m->dim}};
        for (int i = 0; i < 6; i++) {
            if (!fl[i].dst) continue;
            snprintf(nm, sizeof nm, "blk.%d.%s", l, fl[i].sfx);
            t = find_t(ti, nt, nm);
            if (!t) FAIL("missing %s", nm);   /* the reference would read uninitialised memory */
            float* f = load_float(t, base, fl[i].n);
            if (!f) FAIL("cannot load %s", nm);
            memcpy(fl[i].dst, f, (size_t)fl[i].n * 4);
            free(f);
        }
        struct { const char* sfx; qt_t* q; int rows, cols; } ql[7] = {
            {"attn_q.weight", &m->wq[l], m->q_dim, m->dim}, {"attn_k.weight", &m->wk[l], m->kv_dim, m->dim},
            {"attn_v.weight", &m->wv[l], m->kv_dim, m->dim}, {"attn_output.weight", &m->wo[l], m->dim, m->q_dim},
            {"ffn_gate.weight", &m->w1[l], m->hidden, m->dim}, {"ffn_down.weight", &m->w2[l], m->dim, m->hidden},
            {"ffn_up.weight", &m->w3[l], m->hidden, m->dim}};
        for (int i = 0; i < 7; i++) {
            snprintf(nm, sizeof nm, "blk.%d.%s", l, ql[i].sfx);
            t = find_t(ti, nt, nm);
            if (!t) FAIL("missing %s", nm);
            ql[i].q->data = base + t->off; ql[i].q->type = (int)t->type;
            ql[i].q->rows = ql[i].rows; ql[i].q->cols = ql[i].cols;
            ql[i].q->rb = l3o_row_bytes((int)t->type, ql[i].cols);
        }
    }
    t = find_t(ti, nt, "output_norm.weight");
    if (!t || !(m->final_norm = load_float(t, base, m->dim))) FAIL("missing output_norm.weight");
    t = find_t(ti, nt, "output.weight");
    if (t) {
        m->wcls.data = base + t->off; m->wcls.type = (int)t->type;
    } else {                                                                /* tied, c:3064-3079 */
        m->wcls.data = m->emb.data; m->wcls.type = m->emb.type;
    }
    m->wcls.rows = m->vocab; m->wcls.cols = m->dim; m->wcls.rb = l3o_row_bytes(m->wcls.type, m->dim);

    /* run state (c:346-468) */
    int S = m->seq_len;
    m->hq8 = hs / 32 * 34;
    m->head_seq = (size_t)S * m->hq8;
    m->layer_kv = (size_t)m->n_kv * m->head_seq;
    m->attn_scale = 1.0f / sqrtf((float)hs);
    m->embed_scale = sqrtf((float)m->dim);
    m->inv_dim = 1.0f / (float)m->dim;
    m->inv_hs = 1.0f / (float)hs;
    int maxin = m->dim > m->q_dim ? m->dim : m->q_dim;
    if (m->hidden > maxin) maxin = m->hidden;
    m->x = (float*)calloc(m->dim, 4); m->xb = (float*)calloc(m->max_dim, 4); m->xb2 = (float*)calloc(m->dim, 4);
    m->hb = (float*)calloc(m->hidden, 4); m->hb2 = (float*)calloc(m->hidden, 4);
    m->q = (float*)calloc(m->q_dim, 4); m->k = (float*)calloc(m->kv_dim, 4); m->v = (float*)calloc(m->kv_dim, 4);
    m->att = (float*)calloc((size_t)m->n_heads * S, 4); m->logits = (float*)calloc(m->vocab, 4);
    m->kc = (uint8_t*)calloc((size_t)L * m->layer_kv, 1); m->vc = (uint8_t*)calloc((size_t)L * m->layer_kv, 1);
    m->qq8 = (uint8_t*)calloc((size_t)m->n_heads * m->hq8, 1);
    m->xq8 = (uint8_t*)calloc((size_t)(maxin / 32 + 1) * 34, 1);
    int half = hs / 2;
    float* fr = (float*)malloc((size_t)half * 4);
    float* frs = (float*)malloc((size_t)half * 4);
    m->cos_d = (float*)malloc((size_t)S * half * 4); m->sin_d = (float*)malloc((size_t)S * half * 4);
    if (!m->x || !m->xb || !m->kc || !m->vc || !m->att || !m->logits || !fr || !frs || !m->cos_d || !m->sin_d)
        FAIL("out of memory for run state");
    float tswa = m->theta_swa > 0 ? m->theta_swa : 10000.0f;
    for (int i = 0; i < half; i++) {
        fr[i] = 1.0f / powf(m->theta, (float)(i * 2) / (float)hs);
        frs[i] = 1.0f / powf(tswa, (float)(i * 2) / (float)hs);
    }
    for (int p = 0; p < S; p++)
        for (int i = 0; i < half; i++) {
            float a = p * fr[i];
            m->cos_d[(size_t)p * half + i] = cosf(a);
            m->sin_d[(size_t)p * half + i] = sinf(a);
        }
    if (m->is_gemma) {
        m->cos_s = (float*)malloc((size_t)S * half * 4); m->sin_s = (float*)malloc((size_t)S * half * 4);
        if (!m->cos_s || !m->sin_s) FAIL("out of memory for rope tables");
        for (int p = 0; p < S; p++)
            for (int i = 0; i < half; i++) {
                float a = p * frs[i];
                m->cos_s[(size_t)p * half + i] = cosf(a);
                m->sin_s[(size_t)p * half + i] = sinf(a);
            }
    } else {
        m->cos_s = m->cos_d; m->sin_s = m->sin_d;
    }
    free(fr); free(frs);
    free(kv); free(ti);
    return m;
fail:
    free(kv); free(ti);
    l3o_model_close(m);
    return NULL;
}

void l3o_model_close(l3o_model* m) {
    if (!m) return;
    free(m->att_norm); free(m->ffn_norm); free(m->final_norm); free(m->q_norm); free(m->k_norm);
    free(m->post_att_norm); free(m->post_ffn_norm);
    free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->w1); free(m->w2); free(m->w3);
    free(m->x); free(m->xb); free(m->xb2); free(m->hb); free(m->hb2); free(m->q); free(m->k); free(m->v);
    free(m->att); free(m->logits); free(m->kc); free(m->vc); free(m->qq8); free(m->xq8);
    if (m->cos_s != m->cos_d) { free(m->cos_s); free(m->sin_s); }
    free(m->cos_d); free(m->sin_d);
    free(m);
}

void l3o_model_info(const l3o_model* m, int* o) {
    o[0] = m->dim; o[1] = m->hidden; o[2] = m->n_layers; o[3] = m->n_heads; o[4] = m->n_kv;
    o[5] = m->vocab; o[6] = m->seq_len; o[7] = m->head_dim; o[8] = m->is_gemma;
    o[9] = m->swa_window; o[10] = m->swa_pattern;
}

/* The Q8_0-activation dot the reference's matmul_quantized_preq8 (c:2275-2288)
 * calls through a matrix's q8_func when the first matrix of its group (wq,
 * or w1) takes the Q8_0 path; null for a type this restatement lacks. */
typedef float (*q8dot_t)(const uint8_t*, const uint8_t*, int);
static q8dot_t q8_dot_of(int type) {
    switch (type) {
    case L3O_Q4_0: return dot_q4_0_q8_0;
    case L3O_Q4_1: return dot_q4_1_q8_0;
    case L3O_Q5_0: return dot_q5_0_q8_0;
    case L3O_Q5_1: return dot_q5_1_q8_0;
    case L3O_Q8_0: return dot_q8_0_q8_0;
    case L3O_IQ4_NL: return dot_iq4_nl_q8_0;
    default: return 0;
    }
}

static int is_q8_class(int type) { return is_q8_act(type); }   /* q8_func && !deq_func, c:3221 */

static int mm(const qt_t* q, const float* x, float* y) {
    return l3o_matmul(q->type, q->data, q->rows, q->cols, x, y);
}

/* matmul_quantized_preq8 (c:2275-2288): the rows of one matrix dotted with an
 * activation already quantized to Q8_0, through the matrix's own q8 dot. */
static int preq8_rows(const qt_t* w, const uint8_t* xq8, float* out) {
    q8dot_t dot = q8_dot_of(w->type);
    if (!dot) return -1;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < w->rows; r++) out[r] = dot(xq8, w->data + (size_t)r * w->rb, w->cols);
    return 0;
}

/* Q8_0 KV cache dot (c:1574-1597): sum += da*db*(float)isum per block. */
static float kv_dot(const uint8_t* a, const uint8_t* b, int n) {
    float sum = 0.0f;
    for (int i = 0; i < n / 32; i++, a += 34, b += 34) {
        float da = h2f(a), db = h2f(b);
        const int8_t* aq = (const int8_t*)(a + 2);
        const int8_t* bq = (const int8_t*)(b + 2);
        int isum = 0;
        for (int j = 0; j < 32; j++) isum += aq[j] * bq[j];
        sum += da * db * (float)isum;
    }
    return sum;
}

/* Weighted Q8_0 value accumulation (c:1600-1622). */
static void kv_accum(float* out, const uint8_t* c, float w, int n) {
    if (w > -1e-8f && w < 1e-8f) return;
    for (int i = 0; i < n / 32; i++, c += 34) {
        float sc = h2f(c) * w;
        const int8_t* q = (const int8_t*)(c + 2);
        for (int j = 0; j < 32; j++) out[32 * i + j] += q[j] * sc;
    }
}

/* One head's attention over n cache rows (c:3323-3359): scores are the
 * exact Q8_0 dots (dot_q8_0_q8_0_cache, c:1574-1597); with cap > 0 each
 * becomes cap * tanhf(s / cap) (attention logit soft-capping, a load option
 * the reference does not have); softmax (c:3167-3186) into att; out +=
 * sum_t att[t] * V_t (accum_q8_0_cache, c:1600-1622). */
void l3o_attend_head(const uint8_t* q8, const uint8_t* kc, const uint8_t* vc, int n, int hs, float cap,
                     float* att, float* out) {
    int hq8 = hs / 32 * 34;
    for (int t = 0; t < n; t++) {
        float sc = kv_dot(q8, kc + (size_t)t * hq8, hs);
        att[t] = cap > 0.0f ? cap * tanhf(sc / cap) : sc;
    }
    l3o_softmax(att, n);
    for (int t = 0; t < n; t++) kv_accum(out, vc + (size_t)t * hq8, att[t], hs);
}

int l3o_set_attention(l3o_model* m, int swa_pattern, float attn_softcap) {
    if (swa_pattern < 0 || !(attn_softcap >= 0.0f) || isinf(attn_softcap)) return -1;
    if (swa_pattern > 0) m->swa_pattern = swa_pattern;
    m->attn_softcap = attn_softcap;
    return 0;
}

static int swa_layer(const l3o_model* m, int l) {
    return m->swa_pattern > 0 && (l % m->swa_pattern < m->swa_pattern - 1);
}

/* Per-token middle of a layer: QK-norm, RoPE, KV write, attention into out
 * (c:3232-3359 decode; c:3500-3604 prefill, same arithmetic). */
static void attend(l3o_model* m, int l, int pos, float* q, float* k, const float* v, float* out) {
    int hs = m->hs, half = hs / 2;
    float eps = m->eps > 0 ? m->eps : 1e-5f;
    if (m->is_gemma) {
        for (int h = 0; h < m->n_heads; h++)
            rmsnorm_inv(q + h * hs, q + h * hs, m->q_norm + (size_t)l * hs, hs, m->inv_hs, eps);
        for (int h = 0; h < m->n_kv; h++)
            rmsnorm_inv(k + h * hs, k + h * hs, m->k_norm + (size_t)l * hs, hs, m->inv_hs, eps);
    }
    int swa = swa_layer(m, l);
    const float* rc = (m->is_gemma && swa ? m->cos_s : m->cos_d) + (size_t)pos * half;
    const float* rs = (m->is_gemma && swa ? m->sin_s : m->sin_d) + (size_t)pos * half;
    float sc = m->attn_scale;
    if (m->is_gemma) {                                         /* NEOX pairs (i, i+half) */
        for (int h = 0; h < m->n_heads; h++) {
            float* qh = q + h * hs;
            for (int i = 0; i < half; i++) {
                float c = rc[i], s = rs[i], v0 = qh[i], v1 = qh[i + half];
                qh[i] = (v0 * c - v1 * s) * sc;
                qh[i + half] = (v0 * s + v1 * c) * sc;
            }
        }
        for (int h = 0; h < m->n_kv; h++) {
            float* kh = k + h * hs;
            for (int i = 0; i < half; i++) {
                float c = rc[i], s = rs[i], v0 = kh[i], v1 = kh[i + half];
                kh[i] = v0 * c - v1 * s;
                kh[i + half] = v0 * s + v1 * c;
            }
        }
    } else {                                                   /* interleaved pairs */
        for (int i = 0; i < m->q_dim; i += 2) {
            int fi = (i % hs) / 2;
            float c = rc[fi], s = rs[fi], v0 = q[i], v1 = q[i + 1];
            q[i] = (v0 * c - v1 * s) * sc;
            q[i + 1] = (v0 * s + v1 * c) * sc;
            if (i < m->kv_dim) {
                float k0 = k[i], k1 = k[i + 1];
                k[i] = k0 * c - k1 * s;
                k[i + 1] = k0 * s + k1 * c;
            }
        }
    }
    size_t loff = (size_t)l * m->layer_kv;
    for (int h = 0; h < m->n_kv; h++) {
        size_t off = loff + h * m->head_seq + (size_t)pos * m->hq8;
        l3o_quantize_q8_0(k + h * hs, m->kc + off, hs);
        l3o_quantize_q8_0(v + h * hs, m->vc + off, hs);
    }
    l3o_quantize_q8_0(q, m->qq8, m->q_dim);
    memset(out, 0, (size_t)m->q_dim * 4);
    int t0 = 0;
    if (m->is_gemma && swa && m->swa_window > 0) {
        t0 = pos - m->swa_window + 1;
        if (t0 < 0) t0 = 0;
    }
    int na = pos - t0 + 1;
    /* query heads are independent (the reference spreads KV heads over
     * threads, c:3328) */
#pragma omp parallel for schedule(static)
    for (int h = 0; h < m->n_heads; h++) {
        int kh = h / m->kv_mul;
        const uint8_t* kb = m->kc + loff + kh * m->head_seq;
        const uint8_t* vb = m->vc + loff + kh * m->head_seq;
        float* att = m->att + (size_t)h * m->seq_len;
        l3o_attend_head(m->qq8 + h * m->hq8, kb + (size_t)t0 * m->hq8, vb + (size_t)t0 * m->hq8, na, hs,
                        m->attn_softcap, att, out + h * hs);
    }
}

static void ffn_act(const l3o_model* m, float* hb, const float* hb2) {
    if (m->is_gemma) l3o_geglu(hb, hb2, m->hidden);
    else l3o_swiglu(hb, hb2, m->hidden);
}

static void accum(float* a, const float* b, int n) { for (int i = 0; i < n; i++) a[i] += b[i]; }

/* transformer() (c:3190-3435). */
int l3o_forward(l3o_model* m, int token, int pos, int compute_logits, float* logits) {
    if (token < 0 || token >= m->vocab || pos < 0 || pos >= m->seq_len) return -1;
    int dim = m->dim;
    float eps = m->eps > 0 ? m->eps : 1e-5f;
    float* x = m->x;
    if (l3o_dequant_row(m->emb.type, m->emb.data + (size_t)token * m->emb.rb, x, dim)) return -1;
    for (int l = 0; l < m->n_layers; l++) {
        if (m->is_gemma && l == 0) {                                   /* c:3132-3148 */
            float ss = 0.0f;
            for (int j = 0; j < dim; j++) { float xv = x[j] * m->embed_scale; x[j] = xv; ss += xv * xv; }
            ss = 1.0f / sqrtf(ss * m->inv_dim + eps);
            for (int j = 0; j < dim; j++) m->xb[j] = m->att_norm[j] * (ss * x[j]);
        } else {
            rmsnorm_inv(m->xb, x, m->att_norm + (size_t)l * dim, dim, m->inv_dim, eps);
        }
        if (is_q8_class(m->wq[l].type)) {
            /* one Q8_0 quantization shared by q/k/v (c:3221-3225) */
            l3o_quantize_q8_0(m->xb, m->xq8, m->wq[l].cols);
            if (preq8_rows(&m->wq[l], m->xq8, m->q) || preq8_rows(&m->wk[l], m->xq8, m->k) ||
                preq8_rows(&m->wv[l], m->xq8, m->v))
                return -2;
        } else {
            if (mm(&m->wq[l], m->xb, m->q) || mm(&m->wk[l], m->xb, m->k) || mm(&m->wv[l], m->xb, m->v)) return -2;
        }
        attend(m, l, pos, m->q, m->k, m->v, m->xb);
        if (mm(&m->wo[l], m->xb, m->xb2)) return -2;
        if (m->is_gemma) rmsnorm_inv(m->xb2, m->xb2, m->post_att_norm + (size_t)l * dim, dim, m->inv_dim, eps);
        accum(x, m->xb2, dim);
        rmsnorm_inv(m->xb, x, m->ffn_norm + (size_t)l * dim, dim, m->inv_dim, eps);
        if (is_q8_class(m->w1[l].type)) {
            l3o_quantize_q8_0(m->xb, m->xq8, m->w1[l].cols);
            if (preq8_rows(&m->w1[l], m->xq8, m->hb) || preq8_rows(&m->w3[l], m->xq8, m->hb2)) return -2;
        } else {
            if (mm(&m->w1[l], m->xb, m->hb) || mm(&m->w3[l], m->xb, m->hb2)) return -2;
        }
        ffn_act(m, m->hb, m->hb2);
        if (mm(&m->w2[l], m->hb, m->xb)) return -2;
        if (m->is_gemma) rmsnorm_inv(m->xb, m->xb, m->post_ffn_norm + (size_t)l * dim, dim, m->inv_dim, eps);
        accum(x, m->xb, dim);
    }
    rmsnorm_inv(x, x, m->final_norm, dim, m->inv_dim, eps);
    if (compute_logits) {
        if (mm(&m->wcls, x, m->logits)) return -2;
        if (m->is_gemma && m->softcap > 0.0f)
            for (int i = 0; i < m->vocab; i++) m->logits[i] = m->softcap * l3o_fast_tanhf(m->logits[i] / m->softcap);
        if (logits) memcpy(logits, m->logits, (size_t)m->vocab * 4);
    }
    return 0;
}

/* transformer_prefill() (c:3439-3680).  Every batched matmul equals the
 * per-token matmul (see l3o_matmul_batch), so the prefill is the decode
 * layer arithmetic run layer-major over the batch, without logits. */
int l3o_prefill(l3o_model* m, const int* tokens, int start, int bs) {
    int dim = m->dim, md = m->max_dim;
    float eps = m->eps > 0 ? m->eps : 1e-5f;
    if (bs <= 0 || start < 0 || start + bs > m->seq_len) return -1;
    float* bx = (float*)malloc((size_t)bs * dim * 4);
    float* bxb = (float*)calloc((size_t)bs * md, 4);
    float* bxb2 = (float*)malloc((size_t)bs * dim * 4);
    float* bq = (float*)malloc((size_t)bs * m->q_dim * 4);
    float* bk = (float*)malloc((size_t)bs * m->kv_dim * 4);
    float* bv = (float*)malloc((size_t)bs * m->kv_dim * 4);
    float* bh = (float*)malloc((size_t)bs * m->hidden * 4);
    float* bh2 = (float*)malloc((size_t)bs * m->hidden * 4);
    int rc = -1;
    if (!bx || !bxb || !bxb2 || !bq || !bk || !bv || !bh || !bh2) goto out;
    for (int b = 0; b < bs; b++) {
        int tok = tokens[start + b];
        if (tok < 0 || tok >= m->vocab) goto out;
        l3o_dequant_row(m->emb.type, m->emb.data + (size_t)tok * m->emb.rb, bx + (size_t)b * dim, dim);
    }
    for (int l = 0; l < m->n_layers; l++) {
        for (int b = 0; b < bs; b++) {
            float* x = bx + (size_t)b * dim;
            float* o = bxb + (size_t)b * md;
            if (m->is_gemma && l == 0) {
                float ss = 0.0f;
                for (int j = 0; j < dim; j++) { float xv = x[j] * m->embed_scale; x[j] = xv; ss += xv * xv; }
                ss = 1.0f / sqrtf(ss * m->inv_dim + eps);
                for (int j = 0; j < dim; j++) o[j] = m->att_norm[j] * (ss * x[j]);
            } else {
                rmsnorm_inv(o, x, m->att_norm + (size_t)l * dim, dim, m->inv_dim, eps);
            }
        }
        rc = -2;
        if (l3o_matmul_batch(m->wq[l].type, m->wq[l].data, m->q_dim, dim, bxb, bs, md, bq, m->q_dim) ||
            l3o_matmul_batch(m->wk[l].type, m->wk[l].data, m->kv_dim, dim, bxb, bs, md, bk, m->kv_dim) ||
            l3o_matmul_batch(m->wv[l].type, m->wv[l].data, m->kv_dim, dim, bxb, bs, md, bv, m->kv_dim))
            goto out;
        for (int b = 0; b < bs; b++)
            attend(m, l, start + b, bq + (size_t)b * m->q_dim, bk + (size_t)b * m->kv_dim,
                   bv + (size_t)b * m->kv_dim, bxb + (size_t)b * md);
        if (l3o_matmul_batch(m->wo[l].type, m->wo[l].data, dim, m->q_dim, bxb, bs, md, bxb2, dim)) goto out;
        for (int b = 0; b < bs; b++) {
            float* x2 = bxb2 + (size_t)b * dim;
            if (m->is_gemma) rmsnorm_inv(x2, x2, m->post_att_norm + (size_t)l * dim, dim, m->inv_dim, eps);
            accum(bx + (size_t)b * dim, x2, dim);
        }
        for (int b = 0; b < bs; b++)
            rmsnorm_inv(bxb + (size_t)b * md, bx + (size_t)b * dim, m->ffn_norm + (size_t)l * dim, dim, m->inv_dim, eps);
        if (l3o_matmul_batch(m->w1[l].type, m->w1[l].data, m->hidden, dim, bxb, bs, md, bh, m->hidden) ||
            l3o_matmul_batch(m->w3[l].type, m->w3[l].data, m->hidden, dim, bxb, bs, md, bh2, m->hidden))
            goto out;
        for (int b = 0; b < bs; b++) ffn_act(m, bh + (size_t)b * m->hidden, bh2 + (size_t)b * m->hidden);
        if (l3o_matmul_batch(m->w2[l].type, m->w2[l].data, dim, m->hidden, bh, bs, m->hidden, bxb, md)) goto out;
        for (int b = 0; b < bs; b++) {
            float* o = bxb + (size_t)b * md;
            if (m->is_gemma) rmsnorm_inv(o, o, m->post_ffn_norm + (size_t)l * dim, dim, m->inv_dim, eps);
            accum(bx + (size_t)b * dim, o, dim);
        }
    }
    rc = 0;
out:
    free(bx); free(bxb); free(bxb2); free(bq); free(bk); free(bv); free(bh); free(bh2);
    return rc;
}

int l3o_copy_kv(const l3o_model* m, int layer, int which_v, void* dst, size_t cap) {
    if (layer < 0 || layer >= m->n_layers || cap < m->layer_kv) return -1;
    memcpy(dst, (which_v ? m->vc : m->kc) + (size_t)layer * m->layer_kv, m->layer_kv);
    return 0;
}

/* Test support, no counterpart in the reference: overwrite one layer's K or
 * V cache with n bytes (the layout l3o_copy_kv returns), so a long context
 * can be installed without prefilling it here. */
int l3o_set_kv(l3o_model* m, int layer, int which_v, const void* src, size_t n) {
    if (layer < 0 || layer >= m->n_layers || n != m->layer_kv) return -1;
    memcpy((which_v ? m->vc : m->kc) + (size_t)layer * m->layer_kv, src, n);
    return 0;
}

int l3o_rope_row(const l3o_model* m, int swa, int pos, float* c, float* s) {
    if (pos < 0 || pos >= m->seq_len) return -1;
    size_t half = (size_t)m->hs / 2;
    memcpy(c, (swa ? m->cos_s : m->cos_d) + (size_t)pos * half, half * 4);
    memcpy(s, (swa ? m->sin_s : m->sin_d) + (size_t)pos * half, half * 4);
    return 0;
}

int l3o_copy_x(const l3o_model* m, float* dst) {
    memcpy(dst, m->x, (size_t)m->dim * 4);
    return 0;
}
