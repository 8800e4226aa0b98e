// Per-row quantizer shared by the act-quant kernels (act_quant.hip) and the
// fused norm / modulate / quantize kernels (norm_quant.hip).
#pragma once

#include "h3q_common.hpp"

namespace h3q {

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_abs_max(uint32_t acc, uint32_t w) {
    us2 a = __builtin_bit_cast(us2, acc);
    us2 b = __builtin_bit_cast(us2, w & 0x7FFF7FFFu);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}

__device__ __forceinline__ float amax_from_packed(uint32_t m) {
    uint32_t hi = m >> 16, lo = m & 0xFFFFu;
    return __uint_as_float((hi > lo ? hi : lo) << 16);
}

// Integral-valued float -> int clamped to [lo, 127].  v_cvt_i32_f32 is used
// directly for its defined NaN -> 0 and saturating behaviour (a C++ float to
// int conversion of NaN or of an out-of-range value is undefined).
__device__ __forceinline__ int sat_int(float v, int lo) {
    int i;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(v));
    return i < lo ? lo : (i > 127 ? 127 : i);
}

// One row element -> code, for each quantizer form.
template <int FMT, int ROUND>
struct RowQuant {
    float s, r;  // DIV: scale and RN(1/scale); RCP: scale and 127/amax
    __device__ __forceinline__ void init(float amax) {
        if (ROUND == kRoundRcpMul) {
            s = amax / kInt8Max;
            r = (amax == 0.0f) ? 0.0f : kInt8Max / amax;
        } else {
            s = amax_scale(amax, FMT == kFmtE4M3 ? kE4M3Recip : kInt8Recip);
            r = 1.0f / s;
        }
    }
    __device__ __forceinline__ float value(float f) const {
        if (ROUND == kRoundRcpMul) return __builtin_rintf(f * r);
        float q = copysignf(div_rn(f, s, r), f);
        return FMT == kFmtE4M3 ? q : __builtin_rintf(q);
    }
    // 4 bf16 (two packed words) -> 4 code bytes.
    __device__ __forceinline__ uint32_t pack4(uint32_t w0, uint32_t w1) const {
        float a = value(bf16_lo(w0)), b = value(bf16_hi(w0));
        float c = value(bf16_lo(w1)), d = value(bf16_hi(w1));
        if (FMT == kFmtE4M3) {
            a = __builtin_amdgcn_fmed3f(a, -kE4M3Max, kE4M3Max);
            b = __builtin_amdgcn_fmed3f(b, -kE4M3Max, kE4M3Max);
            c = __builtin_amdgcn_fmed3f(c, -kE4M3Max, kE4M3Max);
            d = __builtin_amdgcn_fmed3f(d, -kE4M3Max, kE4M3Max);
            return cvt_e4m3x2(a, b) | (cvt_e4m3x2(c, d) << 16);
        }
        // Saturating convert: v_cvt_i32_f32 maps NaN to 0 and +-inf to the
        // int32 limits, then an integer clamp (NaN -> 0, inf -> 127 / lo as
        // in a saturating int8 convert).
        const int lo = (ROUND == kRoundRcpMul) ? -128 : -127;
        const int ia = sat_int(a, lo), ib = sat_int(b, lo), ic = sat_int(c, lo), id = sat_int(d, lo);
        return (uint32_t)(ia & 0xFF) | ((uint32_t)(ib & 0xFF) << 8) | ((uint32_t)(ic & 0xFF) << 16) |
               ((uint32_t)id << 24);
    }
};

}  // namespace h3q
