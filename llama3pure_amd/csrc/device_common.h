// device_common.h — device helpers shared by the kernels of libl3p.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace l3pd {

// fp16 -> fp32 (IEEE, exact).
__device__ __forceinline__ float h2f(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
}

// fp16 -> fp32 exactly as the reference's table (c:547-582): NaN payloads are
// kept without forcing the quiet bit.  A select, no branch.
__device__ __forceinline__ float h2f_exact(uint32_t h) {
    h &= 0xffffu;
    const float special = __uint_as_float(((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13));
    return ((h >> 10) & 31u) == 31u ? special : h2f(h);
}

// Truncating fp32 -> fp16 (c:585-599), without branches: exponents e <= 0
// give the subnormal (m | 0x400) >> (1 - e), which is 0 once the shift
// passes the 11 bits (the reference's e < -10 case; the shift is capped at
// 31), e >= 31 gives infinity, the rest e << 10 | m.
__device__ __forceinline__ uint32_t f2h_trunc(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int e = (int)((b >> 23) & 0xffu) - 112;
    const uint32_t m = (b >> 13) & 0x3ffu;
    const uint32_t sub = (m | 0x400u) >> min(max(1 - e, 0), 31);
    const uint32_t nrm = e >= 31 ? 0x7c00u : (((uint32_t)e << 10) | m);
    return sign | (e <= 0 ? sub : nrm);
}

__device__ __forceinline__ uint32_t shr64(uint32_t lo, uint32_t hi, uint32_t sh) {
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> sh);
}

// fast_expf / fast_tanhf (c:3089-3106); the library is built with
// -ffp-contract=off so these round exactly like the reference's C.
__device__ __forceinline__ float ref_fast_expf(float x) {
    if (x > 10.0f) return 22026.47f;
    if (x < -10.0f) return 0.0f;
    const float x2 = x * x;
    const float x3 = x2 * x;
    const float num = 120.0f + 60.0f * x + 12.0f * x2 + x3;
    const float den = 120.0f - 60.0f * x + 12.0f * x2 - x3;
    return num / den;
}
__device__ __forceinline__ float ref_fast_tanhf(float x) {
    if (x < -4.0f) return -1.0f;
    if (x > 4.0f) return 1.0f;
    const float x2 = x * x;
    return (x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2)))) /
           (135135.0f + x2 * (62370.0f + x2 * (3150.0f + 28.0f * x2)));
}
// SwiGLU (c:3400-3406) and GeGLU (c:3391-3398) of one gate/up pair.
__device__ __forceinline__ float ref_swiglu(float g, float u) {
    const float v = g * (1.0f / (1.0f + ref_fast_expf(-g)));
    return v * u;
}
__device__ __forceinline__ float ref_geglu(float g, float u) {
    const float x = 0.5f * g * (1.0f + ref_fast_tanhf(g * (0.7978845608f + 0.035677408137f * g * g)));
    return x * u;
}

// Q8_0 quantization of 32 values (quantize_row_q8_0, c:1508-1528).
struct QBlock {
    uint32_t dh;   // truncated fp16 scale
    int8_t q[32];
    int sum;       // sum of quants
};
__device__ __forceinline__ void quantize32(const float* v, QBlock& o) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float a = v[j] < 0 ? -v[j] : v[j];
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;
    o.dh = f2h_trunc(d);
    int s = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        int qi = (int)roundf(v[j] * id);
        qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
        o.q[j] = (int8_t)qi;
        s += qi;
    }
    o.sum = s;
}

// Barrier for LDS traffic only: lgkmcnt(0) and s_barrier, with no wait on
// outstanding vector memory (which __syncthreads' release fence adds, LDS
// copies in flight included).  Callers wait for their own copies explicitly.
__device__ __forceinline__ void lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // vmcnt(63) expcnt(7) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ void wait_lgkm() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Cross-lane exchanges in registers (gfx950), instead of ds_bpermute round
// trips through the LDS unit: the value of the partner lane in butterfly step
// M = 32, 16, 8, 4, 2, 1.  M = 32 and 16 use the permlane swaps (partner lane
// ^ 32, lane ^ 16: swap(x, x) returns the lower and the upper lane's value);
// within a row of 16 lanes, M = 8 pairs lane i with 15 - i and M = 4 pairs i
// with 7 - i (DPP row mirrors), M = 2 and 1 are the quad exchanges i ^ 2 and
// i ^ 1.  Every step pairs lanes that differ in bit log2(M) and agree in all
// higher bits, which is all a butterfly reduction or transpose needs.  Call
// with every lane of the wave active.
template <int M>
__device__ __forceinline__ float lane_partner(float v) {
    const int x = __float_as_int(v);
    if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return __int_as_float((__lane_id() & 32) ? r[0] : r[1]);
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return __int_as_float((__lane_id() & 16) ? r[0] : r[1]);
    } else if constexpr (M == 8) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false));   // row_mirror
    } else if constexpr (M == 4) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false));   // row_half_mirror
    } else if constexpr (M == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]
    } else {
        static_assert(M == 1, "butterfly step");
        return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]
    }
}

// lane_partner with a step known once loops are unrolled
__device__ __forceinline__ float lane_partner_m(float v, int m) {
    switch (m) {
    case 32: return lane_partner<32>(v);
    case 16: return lane_partner<16>(v);
    case 8: return lane_partner<8>(v);
    case 4: return lane_partner<4>(v);
    case 2: return lane_partner<2>(v);
    default: return lane_partner<1>(v);
    }
}

// Sum / maximum over the wave (every lane gets the same value: each step adds
// a lane's and its partner's values, a + b in one and b + a in the other).
__device__ __forceinline__ float wave_sum(float v) {
    v += lane_partner<32>(v);
    v += lane_partner<16>(v);
    v += lane_partner<8>(v);
    v += lane_partner<4>(v);
    v += lane_partner<2>(v);
    v += lane_partner<1>(v);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, lane_partner<32>(v));
    v = fmaxf(v, lane_partner<16>(v));
    v = fmaxf(v, lane_partner<8>(v));
    v = fmaxf(v, lane_partner<4>(v));
    v = fmaxf(v, lane_partner<2>(v));
    v = fmaxf(v, lane_partner<1>(v));
    return v;
}
// Maximum over each 32-lane half of the wave.
__device__ __forceinline__ float half_max(float v) {
    v = fmaxf(v, lane_partner<16>(v));
    v = fmaxf(v, lane_partner<8>(v));
    v = fmaxf(v, lane_partner<4>(v));
    v = fmaxf(v, lane_partner<2>(v));
    v = fmaxf(v, lane_partner<1>(v));
    return v;
}

}  // namespace l3pd
