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

// One row element -> code, for each quantizer form.  The scale is always the
// row's own (from the maximum of |x| over the row), which the e4m3 form relies
// on: |x| <= amax and s = max(RN(amax * RN(1/448)), 1e-12) give
// |x / s| <= 448 (1 + 2^-22), which v_cvt_pk_fp8_f32 rounds to 448 (it
// saturates everything up to 464; measured on MI355X), so the reference's
// clamp to +-448 changes no code and is not applied; a NaN quotient stays NaN,
// as torch's clamp leaves it.
template <int FMT, int ROUND>
struct RowQuant {
    // DIV: scale, RN(1/scale) and the divisor of the residual correction;
    // RCP: scale and 127/amax.
    float s, r, dv;
    __device__ __forceinline__ void init(float amax) {
        if (ROUND == kRoundRcpMul) {
            s = amax / kInt8Max;
            r = (amax == 0.0f) ? 0.0f : kInt8Max / amax;
        } else {
            s = amax_scale(amax, FMT == kFmtE4M3 ? kE4M3Recip : kInt8Recip);
            r = 1.0f / s;
            // A row holding an infinity has s = inf and r = 0, where the
            // correction's q0 * s - x would be 0 * inf = NaN although x / s is
            // +-0.  With dv = 0 the correction adds x * 0 to q0 = x * 0: +-0 for
            // a finite x and NaN (inf * 0) for an infinite one, the IEEE
            // quotients.  For a finite s, dv = s.
            dv = s <= 3.402823466e38f ? s : 0.0f;
        }
    }
    __device__ __forceinline__ float value(float f) const {
        if (ROUND == kRoundRcpMul) return __builtin_rintf(f * r);
        const float q = div_rn_signed(f, dv, r);
        return FMT == kFmtE4M3 ? q : __builtin_rintf(q);
    }
    // 4 bf16 (two packed words) -> 4 code bytes.
    __device__ __forceinline__ uint32_t pack4(uint32_t w0, uint32_t w1) const {
        const float a = value(bf16_lo(w0)), b = value(bf16_hi(w0));
        const float c = value(bf16_lo(w1)), d = value(bf16_hi(w1));
        if (FMT == kFmtE4M3) return cvt_e4m3x2(a, b) | (cvt_e4m3x2(c, d) << 16);
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
