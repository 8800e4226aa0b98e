// Scalar arithmetic shared by the device quantizers and by the host-side
// exhaustive check (tests compile this header with g++ and compare every
// (x, amax) pair the quantizers can meet against IEEE division).
#pragma once

#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define H3Q_HD __host__ __device__ __forceinline__
#else
#define H3Q_HD static inline
#endif

namespace h3q {

// Largest finite magnitudes of the code formats and the scale floor used by
// the reference (torch.clamp(min=1.0e-12) applied to a binary32 tensor).
constexpr float kE4M3Max = 448.0f;
constexpr float kInt8Max = 127.0f;
constexpr float kScaleFloor = 1.0e-12f;

// The reciprocals of the limits, rounded to binary32 (RN(1/448), RN(1/127)).
constexpr float kE4M3Recip = 1.0f / 448.0f;
constexpr float kInt8Recip = 1.0f / 127.0f;

// Correctly rounded binary32 quotient x / s from r = RN(1 / s), one residual
// correction (Markstein's division scheme):
//   q0 = RN(x * r)               within one ulp of x / s
//   e  = x - q0 * s              exact, computed by one fused multiply-add
//   q1 = RN(q0 + e * r)          = RN(x / s)
// Every divisor a quantizer uses is amax_scale(amax, RN(1/c)) for a bf16 amax
// and c in {127, 448}, and every dividend is a bf16 value with |x| <= amax;
// the test suite checks q1 == x / s bit for bit over that whole set.
H3Q_HD float div_rn(float x, float s, float r) {
    float q0 = x * r;
    float e = fmaf(-q0, s, x);
    return fmaf(e, r, q0);
}

// The same quotient with the sign of a zero dividend kept, so that no
// copysign has to follow: the residual is formed with the opposite sign,
//   q0 = RN(x * r);  e = q0 * s - x (exact, one fma);  q1 = RN(q0 - e * r),
// the value of div_rn for every nonzero x, and +-0 for x = +-0 (q0 = +-0,
// e = +0, q1 = -0 * r + q0 = q0) where div_rn gives +0.  The test suite
// checks it against IEEE division over the same set, signs included.
H3Q_HD float div_rn_signed(float x, float s, float r) {
    const float q0 = x * r;
    const float e = fmaf(q0, s, -x);
    return fmaf(-e, r, q0);
}

// The same quotient for any binary32 divisor (a static, calibrated scale or
// one rounded to bf16): where the three operations leave a non-finite value
// (the quotient or the reciprocal overflows, s is 0, inf or NaN, x is inf or
// NaN), the IEEE division decides.  The test suite checks that the finite
// results, rounded to bf16 as the per-tensor quantizer rounds them, equal
// those of IEEE division over every bf16 numerator and every bf16 divisor,
// and over a sweep of binary32 divisors.
// (For x = +-0 the correction loses the sign of the zero quotient; the first
// product has it.)
H3Q_HD float div_rn_any(float x, float s, float r) {
    const float q0 = x * r;
    const float q1 = fmaf(fmaf(-q0, s, x), r, q0);
    if (isfinite(q1)) return x == 0.0f ? q0 : q1;
    return x / s;
}

// Scale of a dynamic quantizer from its absolute maximum:
//   s = max(RN(amax * RN(1/limit)), 1e-12)
// The reference writes torch.clamp(amax.float() / limit, min=1.0e-12)
// (H3/inference/w8a8.py:58-61 with limit 127; FL/inference/fused_kernels.py:
// 791-794, 826-829 and fp8.py:259-262 with 448) and evaluates it on the GPU,
// where PyTorch's kernel for a tensor divided by a Python scalar multiplies by
// the binary32 reciprocal of the scalar: measured on MI355X, bit-identical to
// this form for every bf16 amax, while a true division differs for 1,488 (127)
// and 17,468 (448) of the 32,640 finite values.  The reference's Triton
// finalize kernels compute the same product, maximum * (1.0 / LIMIT)
// (FL/inference/fused_kernels.py:155-172, 209-227).
H3Q_HD float amax_scale(float amax, float recip) {
    float s = amax * recip;
    return s < kScaleFloor ? kScaleFloor : s;
}

}  // namespace h3q
