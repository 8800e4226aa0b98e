// Fused SwiGLU + per-token quantization, gfx950: the producer of the fc2 input
// of a DiT MLP (H3/model/layers.py:469-479: F.silu(gate) * up, or the Triton
// fused_swiglu of H3/inference/fused_kernels.py:240-261, 663-677), with the
// activation quantizer of the following W8A8 linear folded in.  For a row
// [gate (F) | up (F)] of bf16:
//
//   e = exp(-gate)                     (exp_f32 below, within 1 ulp of a
//                                       correctly rounded exp)
//   s = bf16(gate / (1 + e))           (IEEE binary32 sum and division: torch's
//                                       silu, x / (1 + exp(-x)), rounded to bf16)
//   y = bf16(s * up)                   (stored if out)
//   codes, s_row = per-token quantization of y   (if codes)
//
// Every binary32 operation is a single IEEE operation in the order written;
// exp_f32 uses only IEEE multiply-adds and ldexp, so a CPU restatement
// reproduces y bit for bit.  The reference's results differ from these only
// where its own exp (the library's, or Triton's) moves the binary32 silu across
// a bf16 rounding boundary.
//
// One wavefront per row, y kept in VGPRs (NV 8-element vectors per lane) for
// the quantizer; gate and up are read in batches of four vectors per lane.
// Per row 4F bytes in, F bytes of codes + 4 bytes of scale out (+ 2F with out).
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"
#include "row_quant.hpp"

#pragma clang fp contract(off)

namespace h3q {

namespace {

// exp(x) in binary32 from IEEE operations only: x = k ln2 + r with
// k = rint(x / ln2) and r reduced by a two-term ln2 (Cody and Waite), then
// the degree-7 Taylor polynomial of e^r in Horner form (|r| <= ln2 / 2, the
// truncation error is below 2e-9 relative), then the exponent k.  Over every
// binary32 x in [-104, 89] it is within 1 ulp of glibc's expf (99.5% equal).
__device__ __forceinline__ float exp_f32(float x) {
    if (x > 0x1.62e430p+6f) return __builtin_inff();  // above ln(FLT_MAX)
    if (x < -0x1.9fe368p+6f) return 0.0f;              // below ln(smallest subnormal / 2)
    const float k = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-k, 0x1.62e430p-1f, x);
    r = __builtin_fmaf(-k, -0x1.05c610p-29f, r);
    float p = 0x1.a01a02p-13f;  // 1/7!
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1.0p-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + exp_f32(-g)); }

// Two gate and two up values (packed bf16) -> two y values (packed bf16).
__device__ __forceinline__ uint32_t swiglu2(uint32_t g, uint32_t u) {
    const uint32_t s = pack_bf16x2(silu_f32(bf16_lo(g)), silu_f32(bf16_hi(g)));
    return pack_bf16x2(bf16_lo(s) * bf16_lo(u), bf16_hi(s) * bf16_hi(u));
}

}  // namespace

template <int FMT, int ROUND, int NV>
__global__ __launch_bounds__(256) void swiglu_quant_kernel(SwigluQuantArgs p) {
    const int lane = threadIdx.x & 63;
    const int nvec = p.half >> 3;
    const int64_t step = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < p.rows; row += step) {
        const uint4* gr = reinterpret_cast<const uint4*>(p.x + row * p.ldx);
        const uint4* ur = reinterpret_cast<const uint4*>(p.x + row * p.ldx + p.half);
        uint4 y[NV];
        uint32_t m = 0;
        constexpr int B = 4;
#pragma unroll
        for (int i0 = 0; i0 < NV; i0 += B) {
            uint4 g[B], u[B];
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const int vec = (i0 + b) * 64 + lane;
                const bool in = i0 + b < NV && vec < nvec;
                g[b] = in ? gr[vec] : make_uint4(0, 0, 0, 0);
                u[b] = in ? ur[vec] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (i0 + b >= NV) break;
                y[i0 + b] = make_uint4(swiglu2(g[b].x, u[b].x), swiglu2(g[b].y, u[b].y), swiglu2(g[b].z, u[b].z),
                                       swiglu2(g[b].w, u[b].w));
                // Materialize the packed result here: without it the compiler
                // interleaves the exp sequences of several vectors and runs
                // out of registers.
                asm volatile("" : "+v"(y[i0 + b].x), "+v"(y[i0 + b].y), "+v"(y[i0 + b].z), "+v"(y[i0 + b].w));
                m = pk_abs_max(m, y[i0 + b].x);
                m = pk_abs_max(m, y[i0 + b].y);
                m = pk_abs_max(m, y[i0 + b].z);
                m = pk_abs_max(m, y[i0 + b].w);
            }
        }
        if (p.out) {
            uint4* orow = reinterpret_cast<uint4*>(p.out + row * p.ldo);
#pragma unroll
            for (int i = 0; i < NV; ++i)
                if (i * 64 + lane < nvec) orow[i * 64 + lane] = y[i];
        }
        if (p.codes == nullptr) continue;
        const float amax = wave_max(amax_from_packed(m));
        RowQuant<FMT, ROUND> rq;
        rq.init(amax);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vec = i * 64 + lane;
            if (vec < nvec) {
                uint2 o;
                o.x = rq.pack4(y[i].x, y[i].y);
                o.y = rq.pack4(y[i].z, y[i].w);
                *reinterpret_cast<uint2*>(p.codes + row * p.ldq + 8 * (int64_t)vec) = o;
            }
        }
        if (lane == 0) p.scales[row] = rq.s;
    }
}

namespace {

template <int FMT, int ROUND, int NV>
hipError_t launch_sq_nv(const SwigluQuantArgs& a, hipStream_t st) {
    constexpr int64_t kBlocks = 1024;
    const int64_t blocks = (a.rows + 3) / 4 < kBlocks ? (a.rows + 3) / 4 : kBlocks;
    hipLaunchKernelGGL((swiglu_quant_kernel<FMT, ROUND, NV>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <int FMT, int ROUND>
hipError_t launch_sq_fmt(const SwigluQuantArgs& a, hipStream_t st) {
    const int nvec = a.half / 8;
    if (nvec <= 128) return launch_sq_nv<FMT, ROUND, 2>(a, st);
    if (nvec <= 256) return launch_sq_nv<FMT, ROUND, 4>(a, st);
    if (nvec <= 512) return launch_sq_nv<FMT, ROUND, 8>(a, st);
    if (nvec <= 1024) return launch_sq_nv<FMT, ROUND, 16>(a, st);
    if (nvec <= 1792) return launch_sq_nv<FMT, ROUND, 28>(a, st);
    return launch_sq_nv<FMT, ROUND, 32>(a, st);
}

}  // namespace

hipError_t launch_swiglu_quant(const SwigluQuantArgs& a, int fmt, int rounding, hipStream_t st) {
    if (fmt == kFmtInt8)
        return rounding == kRoundRcpMul ? launch_sq_fmt<kFmtInt8, kRoundRcpMul>(a, st)
                                        : launch_sq_fmt<kFmtInt8, kRoundDiv>(a, st);
    return launch_sq_fmt<kFmtE4M3, kRoundDiv>(a, st);
}

}  // namespace h3q
