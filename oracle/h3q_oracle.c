/*
 * CPU oracle for the quantized-linear path.  TEST INFRASTRUCTURE ONLY: this
 * library is loaded by tests/, by __graft_entry__.smoke() as the checker and by
 * bench.py's cpu_baseline leg.  The product path never links or calls it.
 *
 * It restates, in plain C with IEEE single/double arithmetic, the arithmetic of
 * the reference's quantizers and scaled GEMMs:
 *
 *   orc_quant_rows_int8_div    H3/inference/w8a8.py:57-63 (_quantize_weight)
 *                              FL/inference/w8a8.py:242-257 (same formula)
 *   orc_quant_rows_e4m3_div    per-token / per-channel e4m3fn: the formula of
 *                              w8a8.py:57-63 with 127 -> 448 and the e4m3fn cast,
 *                              fp32 quotient as in FL/inference/fused_kernels.py:826-834
 *   orc_quant_rows_int8_rcp    vLLM 0.11.1 dynamic_scaled_int8_quant semantics
 *                              (called at H3/inference/w8a8.py:178); third-party,
 *                              parity unpinned against vLLM itself
 *   orc_quant_tensor_e4m3      FL/inference/fused_kernels.py:771-796 (eager) and
 *                              :140-172,230-247 (Triton: bf16 intermediate);
 *                              FL/inference/fp8.py:259-263 (weights)
 *   orc_exp_f32, orc_swiglu    the fused SwiGLU producer's arithmetic: torch's silu
 *                              x / (1 + exp(-x)) rounded to bf16, times up, rounded
 *                              (H3/model/layers.py:469-479; H3/inference/fused_kernels.py:
 *                              240-261), with the kernel's own exp restated
 *   orc_quant_per_head_e4m3    FL/inference/fused_kernels.py:823-877 (eager :826-834;
 *                              Triton :175-227, :250-273): per-(batch, head) scale,
 *                              fp32 quotient
 *   orc_gemm_i8_i32            exact int32 accumulators of cutlass_scaled_mm
 *                              (H3/inference/w8a8.py:179-186)
 *   orc_gemm_e4m3_f64          exact real value of an e4m3 x e4m3 dot product
 *                              (products exact, sums exact in binary64 for K <= 2^20)
 *   orc_gemm_e4m3_mfma         the same dot product under the measured accumulation
 *                              model of the gfx950 FP8 matrix instruction, with a
 *                              bound on its remaining (combination) rounding
 *   orc_quant_tensor_e4m3_typed the same for bf16 / fp16 / fp32 input, eager form in
 *                              the input's dtype (FL/inference/fp8.py:107-113) or Triton form
 *   orc_f16_to_f32, orc_f32_to_f16  IEEE binary16 conversions (round to nearest even)
 *   orc_epilogue_*             s_a * (s_w * float(acc)) [+ bias] -> bf16 RNE (or fp16)
 *   orc_rms_norm_modulate      H3/inference/fused_kernels.py:287-317 (RMSNorm + AdaLN
 *                              modulate) and :319-357 (with the residual gate), with
 *                              the sum-of-squares order and the IEEE rsqrt that the
 *                              gfx950 kernel fixes (the reference's Triton rsqrt is
 *                              approximate: parity with it is unpinned in the last bits)
 *
 * The e4m3fn and bf16 encoders are written from the format definitions (RNE on
 * an exact binary64 value); they are checked against torch's casts by the tests.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

static float f32_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* ------------------------------------------------------------------ bf16 */

ORC_API float orc_bf16_to_f32(uint16_t h) { return f32_from_bits((uint32_t)h << 16); }

/* Round a binary32 value to bfloat16 (round to nearest, ties to even).  The
 * rounding is done on the exact binary64 value: bfloat16 keeps 8 significant
 * bits and the binary32 exponent range, so the quantum is 2^(e-7) for a value
 * with exponent e >= -126 and 2^-133 below. */
ORC_API uint16_t orc_f32_to_bf16(float f) {
    uint32_t b = bits_from_f32(f);
    if (isnan(f)) return (uint16_t)((b >> 16) | 0x40);   /* quiet NaN, sign kept */
    if (isinf(f) || f == 0.0f) return (uint16_t)(b >> 16);
    double a = fabs((double)f);
    int e;
    frexp(a, &e);                 /* a = m * 2^e, m in [0.5,1) -> exponent e-1 */
    int ex = e - 1;
    if (ex < -126) ex = -126;
    double quantum = ldexp(1.0, ex - 7);
    double r = nearbyint(a / quantum) * quantum;   /* exact: power-of-two scaling */
    float rf = (float)r;                           /* exact or overflow to inf */
    uint32_t rb = bits_from_f32(rf) | (b & 0x80000000u);
    return (uint16_t)(rb >> 16);
}

/* ------------------------------------------------------------------ fp16 */

/* IEEE binary16: 1 sign, 5 exponent (bias 15), 10 mantissa bits. */
ORC_API float orc_f16_to_f32(uint16_t h) {
    int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 31) return m ? f32_from_bits(0x7FC00000u | ((uint32_t)s << 31)) : (s ? -INFINITY : INFINITY);
    v = (e == 0) ? ldexp((double)m, -24) : ldexp(1.0 + m / 1024.0, e - 15);
    return (float)(s ? -v : v);
}

/* Round a binary32 value to binary16, to nearest with ties to even, on the
 * exact binary64 value: quantum 2^(e-10) for exponent e >= -14, 2^-24 below;
 * a magnitude that rounds to 2^16 or more overflows to infinity. */
ORC_API uint16_t orc_f32_to_f16(float f) {
    uint16_t sign = (uint16_t)((bits_from_f32(f) >> 16) & 0x8000);
    if (isnan(f)) return (uint16_t)(sign | 0x7E00);
    double a = fabs((double)f);
    if (isinf(f)) return (uint16_t)(sign | 0x7C00);
    if (a == 0.0) return sign;
    int e;
    frexp(a, &e);
    int ex = e - 1;
    if (ex < -14) ex = -14;
    double quantum = ldexp(1.0, ex - 10);
    double r = nearbyint(a / quantum) * quantum;
    if (r >= 65536.0) return (uint16_t)(sign | 0x7C00);
    if (r == 0.0) return sign;
    if (r < ldexp(1.0, -14)) return (uint16_t)(sign | (uint16_t)(r / ldexp(1.0, -24)));
    int er;
    double mr = frexp(r, &er);
    int expo = er - 1;
    int mant = (int)((mr * 2.0 - 1.0) * 1024.0);
    return (uint16_t)(sign | ((expo + 15) << 10) | mant);
}

/* ---------------------------------------------------------------- e4m3fn */

/* OCP float8 e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits, no
 * infinities, S.1111.111 is NaN, largest finite 448, smallest subnormal 2^-9. */
ORC_API float orc_e4m3_to_f32(uint8_t c) {
    int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
    if (e == 15 && m == 7) return NAN;
    double v = (e == 0) ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
    return (float)(s ? -v : v);
}

/* Round to nearest, ties to even, onto the e4m3fn grid.  A magnitude that
 * rounds above 448 has no finite encoding and becomes NaN (0x7F), matching
 * torch's float -> float8_e4m3fn cast (464 rounds to 448, 470 to NaN). */
ORC_API uint8_t orc_f32_to_e4m3(float f) {
    uint8_t sign = (uint8_t)((bits_from_f32(f) >> 24) & 0x80);
    if (isnan(f)) return (uint8_t)(sign | 0x7F);
    double a = fabs((double)f);
    if (isinf(f)) return (uint8_t)(sign | 0x7F);
    if (a == 0.0) return sign;
    int e;
    frexp(a, &e);
    int ex = e - 1;                 /* a in [2^ex, 2^(ex+1)) */
    if (ex < -6) ex = -6;           /* subnormal quantum 2^-9 */
    double quantum = ldexp(1.0, ex - 3);
    double r = nearbyint(a / quantum) * quantum;
    if (r > 448.0) return (uint8_t)(sign | 0x7F);
    if (r == 0.0) return sign;
    uint8_t code;
    if (r < ldexp(1.0, -6)) {
        code = (uint8_t)(r / ldexp(1.0, -9));          /* 1..7 */
    } else {
        int er;
        double mr = frexp(r, &er);                     /* r = mr*2^er, mr in [0.5,1) */
        int expo = er - 1;                             /* r in [2^expo, 2^(expo+1)) */
        int mant = (int)((mr * 2.0 - 1.0) * 8.0);      /* exact: 3 bits */
        code = (uint8_t)(((expo + 7) << 3) | mant);
    }
    return (uint8_t)(sign | code);
}

/* ------------------------------------------------------ row quantization */

static const float kE4M3Max = 448.0f;
static const float kInt8Max = 127.0f;
static const float kScaleFloor = 1.0e-12f;   /* torch.clamp(min=1.0e-12) on fp32 */

/* Scale from an absolute maximum, as the reference's expression
 * clamp(amax.float() / L, min=1e-12) evaluates on the GPU: PyTorch's device
 * kernel for a tensor divided by a Python scalar multiplies by the binary32
 * reciprocal of the scalar, and the reference's Triton finalize kernels write
 * the same product, maximum * (1.0 / LIMIT) (FL/inference/fused_kernels.py:171,
 * 226).  So s = RN(amax * RN(1/L)), floored at 1e-12; a true division
 * amax / L (torch on the CPU) differs in the last bit for about half of the
 * bf16 amax values at L = 448. */
static float amax_scale(float amax, float limit) {
    const float r = 1.0f / limit;
    const float s = amax * r;
    return s < kScaleFloor ? kScaleFloor : s;
}

static float row_amax(const uint16_t* x, int64_t k) {
    float amax = 0.0f;
    for (int64_t j = 0; j < k; ++j) {
        float v = fabsf(orc_bf16_to_f32(x[j]));
        if (v > amax || isnan(v)) amax = v;
    }
    return amax;
}

/* H3/inference/w8a8.py:57-63:
 *   scale = clamp(amax_row(|W|).float() / 127, min=1e-12)   (amax_scale)
 *   q     = int8(clamp(round_half_even(float(W) / scale), -127, 127))
 * bf16 [rows,K] / fp32 [rows,1] promotes to fp32, so the quotient is one
 * correctly rounded binary32 division. */
ORC_API void orc_quant_rows_int8_div(const uint16_t* x, int64_t rows, int64_t k, int64_t ldx,
                                     int8_t* q, int64_t ldq, float* scales) {
    for (int64_t i = 0; i < rows; ++i) {
        const uint16_t* xr = x + i * ldx;
        const float s = amax_scale(row_amax(xr, k), kInt8Max);
        scales[i] = s;
        for (int64_t j = 0; j < k; ++j) {
            float v = nearbyintf(orc_bf16_to_f32(xr[j]) / s);
            if (v < -127.0f) v = -127.0f;
            if (v > 127.0f) v = 127.0f;
            q[i * ldq + j] = (int8_t)v;
        }
    }
}

/* Per-row e4m3fn with an fp32 quotient:
 *   scale = clamp(amax_row / 448, min=1e-12) (amax_scale);  q = e4m3(clamp(float(x)/scale, +-448)) */
ORC_API void orc_quant_rows_e4m3_div(const uint16_t* x, int64_t rows, int64_t k, int64_t ldx,
                                     uint8_t* q, int64_t ldq, float* scales) {
    for (int64_t i = 0; i < rows; ++i) {
        const uint16_t* xr = x + i * ldx;
        const float s = amax_scale(row_amax(xr, k), kE4M3Max);
        scales[i] = s;
        for (int64_t j = 0; j < k; ++j) {
            float v = orc_bf16_to_f32(xr[j]) / s;
            if (v < -kE4M3Max) v = -kE4M3Max;
            if (v > kE4M3Max) v = kE4M3Max;
            q[i * ldq + j] = orc_f32_to_e4m3(v);
        }
    }
}

/* Per-(batch, head) e4m3fn of x [batch, seq, heads, head_dim]
 * (FL/inference/fused_kernels.py:823-877):
 *   scale[b, h] = clamp(amax_{s,d}(|x|).float() / 448, min=1e-12)   (amax_scale)
 *   q = e4m3(clamp(float(x) / scale[b, h], +-448))
 * bf16 [B,S,H,D] / fp32 [B,1,H,1] promotes to fp32: one correctly rounded
 * binary32 division, no bf16 intermediate (the Triton kernel's div_rn). */
ORC_API void orc_quant_per_head_e4m3(const uint16_t* x, int64_t batch, int64_t seq, int64_t heads,
                                     int64_t head_dim, uint8_t* q, float* scales) {
    const int64_t row = heads * head_dim;
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t h = 0; h < heads; ++h) {
            float amax = 0.0f;
            for (int64_t t = 0; t < seq; ++t) {
                float a = row_amax(x + (b * seq + t) * row + h * head_dim, head_dim);
                if (a > amax || isnan(a)) amax = a;
            }
            const float s = amax_scale(amax, kE4M3Max);
            scales[b * heads + h] = s;
            for (int64_t t = 0; t < seq; ++t) {
                const int64_t off = (b * seq + t) * row + h * head_dim;
                for (int64_t d = 0; d < head_dim; ++d) {
                    float v = orc_bf16_to_f32(x[off + d]) / s;
                    if (v < -kE4M3Max) v = -kE4M3Max;
                    if (v > kE4M3Max) v = kE4M3Max;
                    q[off + d] = orc_f32_to_e4m3(v);
                }
            }
        }
    }
}

/* exp(x) as the fused SwiGLU kernel computes it: x = k ln2 + r, k = rint(x / ln2),
 * r reduced with a two-term ln2 (Cody and Waite), degree-7 Taylor polynomial of
 * e^r in Horner form with fused multiply-adds, then ldexp by k.  The constants
 * are binary32 roundings of ln 2, 1/ln 2 and 1/n!.  Pinned against the C
 * library's expf (within 1 ulp). */
ORC_API float orc_exp_f32(float x) {
    if (x > 0x1.62e430p+6f) return INFINITY;
    if (x < -0x1.9fe368p+6f) return 0.0f;
    const float k = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-k, 0x1.62e430p-1f, x);
    r = fmaf(-k, -0x1.05c610p-29f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1.0p-1f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* SwiGLU of rows [gate (half) | up (half)] (bf16 bits, leading dimension ldx):
 *   s = bf16(gate / (1 + exp(-gate)));  y = bf16(s * up)
 * torch's silu on a bf16 tensor computes x / (1 + exp(-x)) in binary32 and
 * rounds to bf16; the product of two bf16 is exact in binary32 and rounded
 * once (H3/model/layers.py:478: F.silu(gate) * up). */
ORC_API void orc_swiglu(const uint16_t* x, int64_t rows, int64_t half, int64_t ldx, uint16_t* y, int64_t ldy) {
    for (int64_t i = 0; i < rows; ++i) {
        for (int64_t j = 0; j < half; ++j) {
            const float g = orc_bf16_to_f32(x[i * ldx + j]);
            const float u = orc_bf16_to_f32(x[i * ldx + half + j]);
            const float s = orc_bf16_to_f32(orc_f32_to_bf16(g / (1.0f + orc_exp_f32(-g))));
            y[i * ldy + j] = orc_f32_to_bf16(s * u);
        }
    }
}

/* vLLM dynamic per-token int8 (third-party semantics, v0.11.1):
 *   scale = amax / 127 (no floor); inv = amax == 0 ? 0 : 127 / amax
 *   q = saturate_int8(round_half_even(float(x) * inv))
 * The saturating convert maps NaN to 0 and +-inf to 127 / -128 (CUDA's
 * cvt.rni.sat.s8.f32); NaN and inf arise when amax < 127 / FLT_MAX, where
 * inv overflows and 0 * inv is NaN. */
ORC_API void orc_quant_rows_int8_rcp(const uint16_t* x, int64_t rows, int64_t k, int64_t ldx,
                                     int8_t* q, int64_t ldq, float* scales) {
    for (int64_t i = 0; i < rows; ++i) {
        const uint16_t* xr = x + i * ldx;
        float amax = row_amax(xr, k);
        scales[i] = amax / kInt8Max;
        float inv = (amax == 0.0f) ? 0.0f : kInt8Max / amax;
        for (int64_t j = 0; j < k; ++j) {
            float v = nearbyintf(orc_bf16_to_f32(xr[j]) * inv);
            if (isnan(v)) v = 0.0f;
            if (v < -128.0f) v = -128.0f;
            if (v > 127.0f) v = 127.0f;
            q[i * ldq + j] = (int8_t)v;
        }
    }
}

/* Per-tensor e4m3fn (FL/inference/fused_kernels.py:771-796, fp8.py:259-263):
 *   scale = clamp(amax_all.float() / 448, min=1e-12)      (0-dim fp32, amax_scale)
 *   q = e4m3(clamp(bf16(float(x) / d), +-448))
 * A bf16 tensor divided by a 0-dim fp32 tensor yields bf16, so the binary32
 * quotient is rounded to bf16 before the e4m3 cast.  The divisor d is the
 * fp32 scale in the reference's Triton kernel (_round_bf16(div_rn(x, s)),
 * :230-247) and in torch on the CPU; torch on the GPU computes in bf16 and
 * casts the divisor, d = bf16(scale) (bf16_divisor != 0; the eager path of
 * the reference on its device, e.g. its weight conversions).  static_scale
 * (nullable) replaces the dynamic scale as in quantize_fp8_e4m3(value, scale). */
ORC_API void orc_quant_tensor_e4m3(const uint16_t* x, int64_t rows, int64_t k, int64_t ldx,
                                   const float* static_scale, int bf16_divisor, uint8_t* q, int64_t ldq,
                                   float* scale_out) {
    float s;
    if (static_scale) {
        s = *static_scale;
    } else {
        float amax = 0.0f;
        for (int64_t i = 0; i < rows; ++i) {
            float a = row_amax(x + i * ldx, k);
            if (a > amax || isnan(a)) amax = a;
        }
        s = amax_scale(amax, kE4M3Max);
    }
    *scale_out = s;
    const float d = bf16_divisor ? orc_bf16_to_f32(orc_f32_to_bf16(s)) : s;
    for (int64_t i = 0; i < rows; ++i) {
        for (int64_t j = 0; j < k; ++j) {
            float v = orc_bf16_to_f32(orc_f32_to_bf16(orc_bf16_to_f32(x[i * ldx + j]) / d));
            if (v < -kE4M3Max) v = -kE4M3Max;
            if (v > kE4M3Max) v = kE4M3Max;
            q[i * ldq + j] = orc_f32_to_e4m3(v);
        }
    }
}

/* Per-tensor e4m3fn of a bf16 (dtype 0), fp16 (1) or fp32 (2) tensor.
 * eager != 0: torch's clamp(x / scale, -448, 448) in x's dtype as evaluated
 * on the GPU (FL/inference/fused_kernels.py:773, FL/inference/fp8.py:107-113):
 * the 0-dim fp32 scale is cast to x's dtype, the quotient is computed in
 * binary32 and rounded to x's dtype (bf16 / fp16; fp32 / fp32 is one IEEE
 * division).  eager == 0: the Triton kernel (:240-246), the binary32
 * quotient by the fp32 scale rounded to bf16, whatever x's dtype.  The scale
 * is clamp(amax(|x|).float() / 448, min=1e-12) as in orc_quant_tensor_e4m3.
 * A NaN quotient (0 / 0 when an fp16 divisor rounds to zero) is the device's
 * canonical positive NaN: torch.clamp keeps it and the float8 cast writes
 * 0x7F. */
static float typed_load(const void* x, int dtype, int64_t i) {
    if (dtype == 0) return orc_bf16_to_f32(((const uint16_t*)x)[i]);
    if (dtype == 1) return orc_f16_to_f32(((const uint16_t*)x)[i]);
    return ((const float*)x)[i];
}

static float typed_round(float v, int mode) {
    if (mode == 1) return orc_bf16_to_f32(orc_f32_to_bf16(v));
    if (mode == 2) return orc_f16_to_f32(orc_f32_to_f16(v));
    return v;
}

ORC_API void orc_quant_tensor_e4m3_typed(const void* x, int dtype, int eager, int64_t rows, int64_t k, int64_t ldx,
                                         const float* static_scale, uint8_t* q, int64_t ldq, float* scale_out) {
    float s;
    if (static_scale) {
        s = *static_scale;
    } else {
        float amax = 0.0f;
        for (int64_t i = 0; i < rows; ++i)
            for (int64_t j = 0; j < k; ++j) {
                float a = fabsf(typed_load(x, dtype, i * ldx + j));
                if (a > amax || isnan(a)) amax = a;
            }
        s = amax_scale(amax, kE4M3Max);
    }
    *scale_out = s;
    const int mode = !eager ? 1 : dtype == 0 ? 1 : dtype == 1 ? 2 : 0;
    const float d = eager ? typed_round(s, mode) : s;
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < k; ++j) {
            const float xv = typed_load(x, dtype, i * ldx + j);
            float v = typed_round(xv / d, mode);
            if (isnan(v)) {
                q[i * ldq + j] = 0x7F;
                continue;
            }
            if (v < -kE4M3Max) v = -kE4M3Max;
            if (v > kE4M3Max) v = kE4M3Max;
            q[i * ldq + j] = orc_f32_to_e4m3(v);
        }
}

/* ----------------------------------------------------------------- GEMMs */

/* acc[m][n] = sum_k a[m][k] * b[n][k], exact in int32 (|acc| <= K*128^2). */
ORC_API void orc_gemm_i8_i32(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                             int32_t* c, int64_t ldc, int64_t m, int64_t n, int64_t k) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t acc = 0;
            const int8_t* ar = a + i * lda;
            const int8_t* br = b + j * ldb;
            for (int64_t t = 0; t < k; ++t) acc += (int32_t)ar[t] * (int32_t)br[t];
            c[i * ldc + j] = (int32_t)acc;
        }
}

/* Exact real value of sum_k e4m3(a[m][k]) * e4m3(b[n][k]).  Each product is a
 * 4-bit by 4-bit significand product scaled by 2^[-18,17]; binary64 holds any
 * sum of up to 2^20 of them without rounding (span < 53 bits). */
ORC_API void orc_gemm_e4m3_f64(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb,
                               double* c, int64_t ldc, int64_t m, int64_t n, int64_t k) {
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = orc_e4m3_to_f32((uint8_t)i);
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            const uint8_t* ar = a + i * lda;
            const uint8_t* br = b + j * ldb;
            for (int64_t t = 0; t < k; ++t) acc += (double)lut[ar[t]] * (double)lut[br[t]];
            c[i * ldc + j] = acc;
        }
}

/* Accumulation model of the gfx950 FP8 matrix instruction
 * (v_mfma_f32_32x32x64_f8f6f4, one instruction per 64 consecutive k), fitted
 * to dot products measured on MI355X (known answers and 98304 random ones):
 *
 *   - products of two e4m3 values are exact;
 *   - the 64 products of one instruction form 8 groups of 8 consecutive k
 *     (k = 8q .. 8q+7).  Inside a group every product is truncated toward
 *     zero to a multiple of 2^(E-13), where E is the largest exponent sum
 *     e_a + e_b over the group's nonzero products (the exponent fields as
 *     encoded: a subnormal counts as 2^-6; the significand product, which
 *     can reach 3.5, does not move E);
 *   - the group sums and the incoming accumulator are then combined in about
 *     binary32 precision (two passes of 4 groups, round to nearest).
 *
 * model[m][n] is the exact sum of the truncated products.  bound[m][n] bounds
 * the combination rounding: at most 9 rounding nodes per instruction (8 group
 * sums and the accumulator), each off by at most one binary32 ulp (2^-23
 * relative) of a partial sum no larger than the running sum of |truncated
 * products|.  (Measured: within 2^-23 of that running sum per instruction.)
 *
 * The groups are those of a kernel whose lanes feed each 8-byte register
 * group with 8 consecutive k starting at a multiple of 8 (zero padding past K
 * changes nothing).  Integer arithmetic: e4m3 values are multiples of 2^-9, so
 * products are integers in units of 2^-18 (< 2^36) and sums fit in int64; a
 * grid of 2^(E-13) is 2^(E+5) units. */
ORC_API void orc_gemm_e4m3_mfma(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb,
                                double* model, double* bound, int64_t ldc, int64_t m, int64_t n, int64_t k) {
    int32_t lut[256], xlut[256];
    for (int i = 0; i < 256; ++i) {
        float v = orc_e4m3_to_f32((uint8_t)i);
        lut[i] = isnan(v) ? 0 : (int32_t)ldexp((double)v, 9);
        const int field = (i >> 3) & 15;
        xlut[i] = (i & 0x7F) == 0 ? -1000 : (field == 0 ? -6 : field - 7);
    }
    const double unit = ldexp(1.0, -18);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            const uint8_t* ar = a + i * lda;
            const uint8_t* br = b + j * ldb;
            int64_t acc = 0, abs_run = 0;
            double rsum = 0.0;
            for (int64_t k0 = 0; k0 < k; k0 += 8) {
                int64_t mag[8];
                int neg[8], emax = -1000;
                const int64_t cnt = (k - k0) < 8 ? (k - k0) : 8;
                for (int64_t t = 0; t < 8; ++t) {
                    int64_t p = 0;
                    if (t < cnt) {
                        const uint8_t ca = ar[k0 + t], cb = br[k0 + t];
                        p = (int64_t)lut[ca] * lut[cb];
                        const int es = xlut[ca] + xlut[cb];
                        if (p != 0 && es > emax) emax = es;
                    }
                    neg[t] = p < 0;
                    mag[t] = p < 0 ? -p : p;
                }
                const int shift = emax + 5 > 0 ? emax + 5 : 0;
                for (int t = 0; t < 8; ++t) {
                    const int64_t q = (mag[t] >> shift) << shift;
                    acc += neg[t] ? -q : q;
                    abs_run += q;
                }
                if (((k0 + 8) & 63) == 0 || k0 + 8 >= k) rsum += 9.0 * (double)abs_run;
            }
            model[i * ldc + j] = (double)acc * unit;
            bound[i * ldc + j] = rsum * unit * ldexp(1.0, -23);
        }
}

/* out = bf16(s_a[m] * (s_w[n] * float(acc)) [+ bias[n]]).  With a bias the
 * final step is one fused multiply-add (the CUTLASS ScaledEpilogueBias order).
 * out_f16 != 0: bias and out are binary16 (torch._scaled_mm(out_dtype=
 * float16, bias=fp16), FL/inference/fp8.py:135-143), one rounding. */
static uint16_t epilogue_one(float acc, float sa, float sw, const uint16_t* bias, int64_t j, int out_f16) {
    float t = sw * acc;
    float v = bias ? fmaf(sa, t, out_f16 ? orc_f16_to_f32(bias[j]) : orc_bf16_to_f32(bias[j])) : sa * t;
    return out_f16 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
}

ORC_API void orc_epilogue_i32(const int32_t* acc, int64_t ldacc, const float* s_a, int s_a_per_row,
                              const float* s_w, int s_w_per_col, const uint16_t* bias,
                              uint16_t* out, int64_t ldo, int64_t m, int64_t n, int out_f16) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j)
            out[i * ldo + j] = epilogue_one((float)acc[i * ldacc + j], s_a[s_a_per_row ? i : 0],
                                            s_w[s_w_per_col ? j : 0], bias, j, out_f16);
}

/* Same epilogue on an exact (binary64) accumulator rounded once to binary32. */
ORC_API void orc_epilogue_f64(const double* acc, int64_t ldacc, const float* s_a, int s_a_per_row,
                              const float* s_w, int s_w_per_col, const uint16_t* bias,
                              uint16_t* out, int64_t ldo, int64_t m, int64_t n, int out_f16) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j)
            out[i * ldo + j] = epilogue_one((float)acc[i * ldacc + j], s_a[s_a_per_row ? i : 0],
                                            s_w[s_w_per_col ? j : 0], bias, j, out_f16);
}

/* ------------------------------------------------- RMSNorm + AdaLN modulate */

/* The reference's _round_bf16 (H3/inference/fused_kernels.py:65-68): add
 * 0x7FFF plus the lowest kept bit to the binary32 bits and truncate. */
static float round_bf16_ref(float f) {
    uint32_t b = bits_from_f32(f);
    return f32_from_bits((b + 0x7FFFu + ((b >> 16) & 1u)) & 0xFFFF0000u);
}

/* For each row r (t = indices[r]):
 *   [branch] h = bf16(residual + bf16(gate[t] * branch))  -> hidden
 *   v = branch ? h : value
 *   ss: 64 lane sums, lane l adding v[8 (l + 64 i) + e]^2 by one fused
 *       multiply-add each (s = fma(v, v, s)) in ascending (i, e); then 6
 *       butterfly steps s_l += s_(l xor d), d = 32, 16, ..., 1
 *   rs = 1 / sqrt(ss / cols + eps)   (each operation an IEEE binary32 operation)
 *   n  = bf16((v * rs) * weight);  y = bf16(bf16(n * bf16(1 + scale[t])) + shift[t])
 * cols must be a multiple of 8.  hidden may be NULL without branch. */
ORC_API void orc_rms_norm_modulate(const uint16_t* value, int64_t ldv, const uint16_t* branch, int64_t ldb,
                                   const uint16_t* gate, const uint16_t* weight, const uint16_t* scale,
                                   const uint16_t* shift, int64_t table_stride, const int64_t* indices,
                                   int64_t rows, int64_t cols, float eps, uint16_t* hidden, int64_t ldh,
                                   uint16_t* out, int64_t ldo) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t t = indices[r];
        float v[8192];
        for (int64_t k = 0; k < cols; ++k) {
            const float x = orc_bf16_to_f32(value[r * ldv + k]);
            if (branch) {
                const float g = orc_bf16_to_f32(gate[t * table_stride + k]);
                const float b = orc_bf16_to_f32(branch[r * ldb + k]);
                const float h = round_bf16_ref(x + round_bf16_ref(g * b));
                v[k] = h;
                if (hidden) hidden[r * ldh + k] = (uint16_t)(bits_from_f32(h) >> 16);
            } else {
                v[k] = x;
            }
        }
        float lane[64];
        const int64_t nvec = cols / 8;
        for (int l = 0; l < 64; ++l) {
            float s = 0.0f;
            for (int64_t vec = l; vec < nvec; vec += 64)
                for (int e = 0; e < 8; ++e) {
                    const float x = v[8 * vec + e];
                    s = fmaf(x, x, s);
                }
            lane[l] = s;
        }
        for (int d = 32; d >= 1; d >>= 1) {
            float nxt[64];
            for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ d];
            memcpy(lane, nxt, sizeof(lane));
        }
        const float mean = lane[0] / (float)cols;
        const float root = sqrtf(mean + eps);
        const float rs = 1.0f / root;
        for (int64_t k = 0; k < cols; ++k) {
            const float w = orc_bf16_to_f32(weight[k]);
            const float sc = orc_bf16_to_f32(scale[t * table_stride + k]);
            const float sh = orc_bf16_to_f32(shift[t * table_stride + k]);
            const float vr = v[k] * rs;
            const float n = round_bf16_ref(vr * w);
            const float one_sc = round_bf16_ref(1.0f + sc);
            const float y = round_bf16_ref(round_bf16_ref(n * one_sc) + sh);
            out[r * ldo + k] = (uint16_t)(bits_from_f32(y) >> 16);
        }
    }
}
