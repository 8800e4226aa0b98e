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

// Correctly rounded binary32 quotient x / s from r = RN(1 / s), one residual
// correction (Markstein's division scheme):
//   q0 = RN(x * r)               within one ulp of x / s
//   e  = x - q0 * s              exact, computed by one fused multiply-add
//   q1 = RN(q0 + e * r)          = RN(x / s)
// Every divisor a row quantizer uses is max(amax / c, 1e-12) for a bf16 amax
// and c in {127, 448}, and every dividend is a bf16 value with |x| <= amax;
// the test suite checks q1 == x / s bit for bit over that whole set.
H3Q_HD float div_rn(float x, float s, float r) {
    float q0 = x * r;
    float e = fmaf(-q0, s, x);
    return fmaf(e, r, q0);
}

// Row scale from the row's absolute maximum (H3/inference/w8a8.py:58-61,
// with limit 127 for int8 codes and 448 for e4m3fn codes).
H3Q_HD float row_scale(float amax, float limit) {
    float s = amax / limit;
    return s < kScaleFloor ? kScaleFloor : s;
}

}  // namespace h3q
