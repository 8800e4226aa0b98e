// Fused RMSNorm + AdaLN modulate (+ residual gate) + per-token quantization,
// gfx950.  The producers of the QKV and fc1 inputs of a DiT block
// (H3/inference/fused_kernels.py:288-357 kernels, 700-773 wrappers), with
// the activation quantizer of the following W8A8 linear folded in:
//
//   [resid] hidden = bf16(residual + bf16(gate[t] * branch))        (stored)
//           v      = resid ? hidden : value
//           rs     = 1 / sqrt(sum(v * v) / cols + eps)
//           n      = bf16((v * rs) * weight)
//           y      = bf16(bf16(n * bf16(1 + scale[t])) + shift[t])  (stored if out)
//           codes, s_row = per-token quantization of y               (if codes)
//
// with t = indices[row] selecting a row of the scale / shift / gate tables.
// Every binary32 operation is a single IEEE round-to-nearest operation in the
// order written (no contraction).  The sum of squares has a fixed order:
// lane l of the row's wavefront accumulates its elements k = 8 (l + 64 i) + e
// in ascending (i, e), then a butterfly over the 64 lanes (xor 32, 16, ..., 1)
// adds the lane partial sums.  rs is the IEEE square root followed by an IEEE
// division.  The reference's Triton kernels use the hardware's approximate
// rsqrt and an unspecified reduction tree, so their rs can differ in the last
// bits; these kernels instead fix both so that a CPU restatement reproduces
// them bit for bit.
//
// One wavefront per row, the row in VGPRs (NV 8-element vectors per lane), so
// the inputs are read from HBM once and y never goes back to memory when only
// the codes are wanted: per row 2 * cols bytes in (4 * cols with the residual
// gate), cols bytes of codes + 4 bytes of scale out (+ 2 * cols for hidden).
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"
#include "row_quant.hpp"

// Every product and sum below is rounded on its own: contraction into FMA is
// off for this file.  (The toolchain's __fadd_rn / __fmul_rn are plain + and
// * compiled in a header where contraction is on, so they are not used.)
#pragma clang fp contract(off)

namespace h3q {

namespace {

// Two binary32 values -> two bf16 in one word (low half first), round to
// nearest even: gfx950's v_cvt_pk_bf16_f32.  For finite values this is the
// reference's _round_bf16 (H3/inference/fused_kernels.py:65-68: add 0x7FFF
// plus the lowest kept bit, truncate), infinities included; NaNs come out as
// NaNs with possibly different payload bits.
__device__ __forceinline__ uint32_t rb2(float lo, float hi) { return pack_bf16x2(lo, hi); }

// Single IEEE binary32 operations, each rounded to nearest even (contraction
// is off in this file, so the compiler keeps them separate).
__device__ __forceinline__ float fadd(float a, float b) { return a + b; }
__device__ __forceinline__ float fmul(float a, float b) { return a * b; }

__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ uint32_t words_of(const uint4& v, int j) {
    return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}

}  // namespace

template <int FMT, int ROUND, int NV, bool RESID>
__global__ __launch_bounds__(256) void norm_modulate_quant_kernel(NormQuantArgs p) {
    const int lane = threadIdx.x & 63;
    const int nvec = p.cols >> 3;
    const int64_t step = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < p.rows; row += step) {
        const int64_t trow = p.indices[row];
        const uint4* tab_scale = reinterpret_cast<const uint4*>(p.scale + trow * p.table_stride);
        const uint4* tab_shift = reinterpret_cast<const uint4*>(p.shift + trow * p.table_stride);
        const uint4* wv = reinterpret_cast<const uint4*>(p.weight);
        uint4 v[NV];
        if constexpr (RESID) {
            const uint4* rr = reinterpret_cast<const uint4*>(p.value + row * p.ldv);
            const uint4* br = reinterpret_cast<const uint4*>(p.branch + row * p.ldb);
            const uint4* gr = reinterpret_cast<const uint4*>(p.gate + trow * p.table_stride);
            uint4* hr = reinterpret_cast<uint4*>(p.hidden + row * p.ldh);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int vec = i * 64 + lane;
                v[i] = make_uint4(0, 0, 0, 0);
                if (vec < nvec) {
                    const uint4 r = rr[vec], b = br[vec], g = gr[vec];
                    uint32_t h[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t rw = words_of(r, j), bw = words_of(b, j), gw = words_of(g, j);
                        const uint32_t gb = rb2(fmul(lo_f(gw), lo_f(bw)), fmul(hi_f(gw), hi_f(bw)));
                        h[j] = rb2(fadd(lo_f(rw), lo_f(gb)), fadd(hi_f(rw), hi_f(gb)));
                    }
                    v[i] = make_uint4(h[0], h[1], h[2], h[3]);
                    hr[vec] = v[i];
                }
            }
        } else {
            const uint4* xr = reinterpret_cast<const uint4*>(p.value + row * p.ldv);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int vec = i * 64 + lane;
                v[i] = vec < nvec ? xr[vec] : make_uint4(0, 0, 0, 0);
            }
        }

        // Sum of squares in the fixed order, then the butterfly.
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (i * 64 + lane < nvec) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = words_of(v[i], j);
                    ss = fadd(ss, fmul(lo_f(w), lo_f(w)));
                    ss = fadd(ss, fmul(hi_f(w), hi_f(w)));
                }
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss = fadd(ss, __shfl_xor(ss, off, 64));
        // The empty asm keeps the compiler from folding 1 / sqrt(.) into one
        // reciprocal-square-root sequence (a different rounding).
        float root = __builtin_sqrtf(fadd(ss / (float)p.cols, p.eps));
        asm volatile("" : "+v"(root));
        const float rs = 1.0f / root;

        // The row stays packed (two bf16 per register) between the passes:
        // without this the compiler keeps the unpacked binary32 values of the
        // sum-of-squares pass alive for reuse, which triples the register
        // footprint and cuts the waves per SIMD from 8 to 2.
#pragma unroll
        for (int i = 0; i < NV; ++i) asm volatile("" : "+v"(v[i].x), "+v"(v[i].y), "+v"(v[i].z), "+v"(v[i].w));

        // Normalize, modulate; y replaces v in registers.  The bf16 output
        // (if any) is stored after this loop, so no store is ordered between
        // the table loads.
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vec = i * 64 + lane;
            if (vec < nvec) {
                const uint4 w = wv[vec], sc = tab_scale[vec], sh = tab_shift[vec];
                uint32_t y[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t xw = words_of(v[i], j), ww = words_of(w, j);
                    const uint32_t cw = words_of(sc, j), hw = words_of(sh, j);
                    const uint32_t nw = rb2(fmul(fmul(lo_f(xw), rs), lo_f(ww)), fmul(fmul(hi_f(xw), rs), hi_f(ww)));
                    const uint32_t s1 = rb2(fadd(1.0f, lo_f(cw)), fadd(1.0f, hi_f(cw)));
                    const uint32_t tw = rb2(fmul(lo_f(nw), lo_f(s1)), fmul(hi_f(nw), hi_f(s1)));
                    y[j] = rb2(fadd(lo_f(tw), lo_f(hw)), fadd(hi_f(tw), hi_f(hw)));
                    m = pk_abs_max(m, y[j]);
                }
                v[i] = make_uint4(y[0], y[1], y[2], y[3]);
            }
        }
        if (p.out) {
            uint4* orow = reinterpret_cast<uint4*>(p.out + row * p.ldo);
#pragma unroll
            for (int i = 0; i < NV; ++i)
                if (i * 64 + lane < nvec) orow[i * 64 + lane] = v[i];
        }
        if (p.codes == nullptr) continue;
#pragma unroll
        for (int i = 0; i < NV; ++i) asm volatile("" : "+v"(v[i].x), "+v"(v[i].y), "+v"(v[i].z), "+v"(v[i].w));

        // Per-token quantization of y, exactly as quant_rows_vec_kernel.
        const float amax = wave_max(amax_from_packed(m));
        RowQuant<FMT, ROUND> rq;
        rq.init(amax);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vec = i * 64 + lane;
            if (vec < nvec) {
                uint2 out;
                out.x = rq.pack4(v[i].x, v[i].y);
                out.y = rq.pack4(v[i].z, v[i].w);
                *reinterpret_cast<uint2*>(p.codes + row * p.ldq + 8 * (int64_t)vec) = out;
            }
        }
        if (lane == 0) p.scales[row] = rq.s;
    }
}

namespace {

template <int FMT, int ROUND, int NV>
hipError_t launch_nq_nv(const NormQuantArgs& a, bool resid, hipStream_t st) {
    constexpr int64_t kBlocks = 1024;
    const int64_t blocks = (a.rows + 3) / 4 < kBlocks ? (a.rows + 3) / 4 : kBlocks;
    if (resid)
        hipLaunchKernelGGL((norm_modulate_quant_kernel<FMT, ROUND, NV, true>), dim3((unsigned)blocks), dim3(256), 0,
                           st, a);
    else
        hipLaunchKernelGGL((norm_modulate_quant_kernel<FMT, ROUND, NV, false>), dim3((unsigned)blocks), dim3(256), 0,
                           st, a);
    return hipGetLastError();
}

template <int FMT, int ROUND>
hipError_t launch_nq_fmt(const NormQuantArgs& a, bool resid, hipStream_t st) {
    const int nvec = a.cols / 8;
    if (nvec <= 128) return launch_nq_nv<FMT, ROUND, 2>(a, resid, st);
    if (nvec <= 256) return launch_nq_nv<FMT, ROUND, 4>(a, resid, st);
    if (nvec <= 512) return launch_nq_nv<FMT, ROUND, 8>(a, resid, st);
    if (nvec <= 704) return launch_nq_nv<FMT, ROUND, 11>(a, resid, st);
    return launch_nq_nv<FMT, ROUND, 16>(a, resid, st);
}

}  // namespace

hipError_t launch_norm_modulate_quant(const NormQuantArgs& a, bool resid, int fmt, int rounding, hipStream_t st) {
    if (fmt == kFmtInt8)
        return rounding == kRoundRcpMul ? launch_nq_fmt<kFmtInt8, kRoundRcpMul>(a, resid, st)
                                        : launch_nq_fmt<kFmtInt8, kRoundDiv>(a, resid, st);
    return launch_nq_fmt<kFmtE4M3, kRoundDiv>(a, resid, st);
}

}  // namespace h3q
