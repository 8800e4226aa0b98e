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
// in ascending (i, e), each by one fused multiply-add (ss = fma(v, v, ss)),
// then a butterfly over the 64 lanes (xor 32, 16, ..., 1) adds the lane
// partial sums.  rs is the IEEE square root followed by an IEEE
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

// One binary32 value rounded to bf16 and kept as binary32: the same
// conversion with +0 as the low half leaves bf16(v) in the high half and
// zeros below it, which is the binary32 value bf16(v) (one instruction, where
// packing and unpacking again takes one and a half per value).
__device__ __forceinline__ float rb1(float v) { return __uint_as_float(pack_bf16x2(0.0f, v)); }

// Single IEEE binary32 operations, each rounded to nearest even (contraction
// is off in this file, so the compiler keeps them separate).
__device__ __forceinline__ float fadd(float a, float b) { return a + b; }
__device__ __forceinline__ float fmul(float a, float b) { return a * b; }

__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ uint32_t words_of(const uint4& v, int j) {
    return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}

// 16-byte vector `vec` of a buffer of nvec vectors; a lane past the end gets
// an out-of-range offset and reads zeros.  No branch, so the compiler keeps
// every load of a row in flight together (a load under a per-lane condition
// is emitted as a masked load followed by a wait).
__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, int vec, int nvec) {
    const v4u w = __builtin_amdgcn_raw_buffer_load_b128(r, vec < nvec ? vec * 16 : (int)0x80000000u, 0, 0);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// The store counterpart: a lane past the end is dropped by the hardware.
__device__ __forceinline__ void store16(__amdgpu_buffer_rsrc_t r, int vec, int nvec, const uint4& v) {
    __builtin_amdgcn_raw_buffer_store_b128(v4u{v.x, v.y, v.z, v.w}, r, vec < nvec ? vec * 16 : (int)0x80000000u, 0, 0);
}

}  // namespace

template <int FMT, int ROUND, int NV, bool RESID>
__global__ __launch_bounds__(256) void norm_modulate_quant_kernel(NormQuantArgs p) {
    const int lane = threadIdx.x & 63;
    const int nvec = p.cols >> 3;
    const int64_t step = (int64_t)gridDim.x * 4;
    // The row (and every buffer descriptor built from it) is wave-uniform;
    // saying so keeps the descriptors in SGPRs (otherwise each buffer load
    // is wrapped in a loop over the distinct descriptors of the wave).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // The table rows of this wave's next 64 rows are read together (lane l
    // holds that of row + l * step) and picked out with readlane, so a row's
    // loads wait for no index load of their own.
    int idx_lo = 0, idx_hi = 0;
    int it = 0;
    for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < p.rows; row += step, ++it) {
        if ((it & 63) == 0) {
            const int64_t r = row + (int64_t)lane * step;
            const int64_t t = r < p.rows ? p.indices[r] : 0;
            idx_lo = (int)(uint32_t)t;
            idx_hi = (int)(t >> 32);
        }
        const int64_t trow = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane(idx_hi, it & 63) << 32) |
                                       (uint32_t)__builtin_amdgcn_readlane(idx_lo, it & 63));
        const uint32_t row_bytes = (uint32_t)nvec * 16u;
        const __amdgpu_buffer_rsrc_t tab_scale = make_rsrc(p.scale + trow * p.table_stride, row_bytes);
        const __amdgpu_buffer_rsrc_t tab_shift = make_rsrc(p.shift + trow * p.table_stride, row_bytes);
        const __amdgpu_buffer_rsrc_t wv = make_rsrc(p.weight, row_bytes);
        uint4 v[NV];
        if constexpr (RESID) {
            const __amdgpu_buffer_rsrc_t rr = make_rsrc(p.value + row * p.ldv, row_bytes);
            const __amdgpu_buffer_rsrc_t br = make_rsrc(p.branch + row * p.ldb, row_bytes);
            const __amdgpu_buffer_rsrc_t gr = make_rsrc(p.gate + trow * p.table_stride, row_bytes);
            const __amdgpu_buffer_rsrc_t hr = make_rsrc(p.hidden + row * p.ldh, row_bytes);
            // Batches of four vectors (twelve loads in flight).
            constexpr int B = 4;
#pragma unroll
            for (int i0 = 0; i0 < NV; i0 += B) {
                uint4 r[B], b[B], g[B];
#pragma unroll
                for (int k = 0; k < B && i0 + k < NV; ++k) {
                    const int vec = (i0 + k) * 64 + lane;
                    r[k] = load16(rr, vec, nvec);
                    b[k] = load16(br, vec, nvec);
                    g[k] = load16(gr, vec, nvec);
                }
#pragma unroll
                for (int k = 0; k < B && i0 + k < NV; ++k) {
                    const int vec = (i0 + k) * 64 + lane;
                    uint32_t h[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t rw = words_of(r[k], j), bw = words_of(b[k], j), gw = words_of(g[k], j);
                        const uint32_t gb = rb2(fmul(lo_f(gw), lo_f(bw)), fmul(hi_f(gw), hi_f(bw)));
                        h[j] = rb2(fadd(lo_f(rw), lo_f(gb)), fadd(hi_f(rw), hi_f(gb)));
                    }
                    // Past the row the inputs read as zeros, and 0 + bf16(0 * 0) = +0.
                    v[i0 + k] = make_uint4(h[0], h[1], h[2], h[3]);
                    store16(hr, vec, nvec, v[i0 + k]);
                }
            }
        } else {
            const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.value + row * p.ldv, row_bytes);
#pragma unroll
            for (int i = 0; i < NV; ++i) v[i] = load16(xr, i * 64 + lane, nvec);
        }

        // Weight / scale / shift vectors in batches of TB, two batches in
        // registers: batch 0 is requested with the row, batch b + 1 before
        // batch b is used, so the table round trips overlap the arithmetic.
        constexpr int TB = 2;
        uint4 w[2][TB], sc[2][TB], sh[2][TB];
        auto load_tables = [&](int i0, int slot) {
#pragma unroll
            for (int k = 0; k < TB; ++k) {
                if (i0 + k < NV) {
                    const int vec = (i0 + k) * 64 + lane;
                    w[slot][k] = load16(wv, vec, nvec);
                    sc[slot][k] = load16(tab_scale, vec, nvec);
                    sh[slot][k] = load16(tab_shift, vec, nvec);
                }
            }
        };
        load_tables(0, 0);
        __builtin_amdgcn_sched_barrier(0);  // issued here, not moved to their first use

        // Sum of squares in the fixed order, then the butterfly.  Lanes past
        // the row hold +0 (read as zeros above), and ss + (+0 * +0) = ss.
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t w = words_of(v[i], j);
                ss = __builtin_fmaf(lo_f(w), lo_f(w), ss);
                ss = __builtin_fmaf(hi_f(w), hi_f(w), ss);
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
        for (int i0 = 0; i0 < NV; i0 += TB) {
            const int slot = (i0 / TB) & 1;
            if (i0 + TB < NV) load_tables(i0 + TB, slot ^ 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < TB && i0 + k < NV; ++k) {
                const int i = i0 + k;
                // Past the row x, w, scale and shift are zeros; with rs = 0
                // there y = bf16(bf16(0 * 1) + 0) = +0 even when rs is infinite.
                const float rsi = i * 64 + lane < nvec ? rs : 0.0f;
                uint32_t y[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t xw = words_of(v[i], j), ww = words_of(w[slot][k], j);
                    const uint32_t cw = words_of(sc[slot][k], j), hw = words_of(sh[slot][k], j);
                    const float n0 = rb1(fmul(fmul(lo_f(xw), rsi), lo_f(ww)));
                    const float n1 = rb1(fmul(fmul(hi_f(xw), rsi), hi_f(ww)));
                    const float t0 = rb1(fmul(n0, rb1(fadd(1.0f, lo_f(cw)))));
                    const float t1 = rb1(fmul(n1, rb1(fadd(1.0f, hi_f(cw)))));
                    y[j] = rb2(fadd(t0, lo_f(hw)), fadd(t1, hi_f(hw)));
                    m = pk_abs_max(m, y[j]);
                }
                v[i] = make_uint4(y[0], y[1], y[2], y[3]);
            }
        }
        if (p.out) {
            const __amdgpu_buffer_rsrc_t orow = make_rsrc(p.out + row * p.ldo, row_bytes);
#pragma unroll
            for (int i = 0; i < NV; ++i) store16(orow, i * 64 + lane, nvec, v[i]);
        }
        if (p.codes == nullptr) continue;
#pragma unroll
        for (int i = 0; i < NV; ++i) asm volatile("" : "+v"(v[i].x), "+v"(v[i].y), "+v"(v[i].z), "+v"(v[i].w));

        // Per-token quantization of y, exactly as quant_rows_vec_kernel.
        const float amax = wave_max(amax_from_packed(m));
        RowQuant<FMT, ROUND> rq;
        rq.init(amax);
        const __amdgpu_buffer_rsrc_t qrow = make_rsrc(p.codes + row * p.ldq, (uint32_t)nvec * 8u);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vec = i * 64 + lane;
            const v2u out = {rq.pack4(v[i].x, v[i].y), rq.pack4(v[i].z, v[i].w)};
            __builtin_amdgcn_raw_buffer_store_b64(out, qrow, vec < nvec ? vec * 8 : (int)0x80000000u, 0, 0);
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
    if (nvec <= 640) return launch_nq_nv<FMT, ROUND, 10>(a, resid, st);  // K = 5120 exactly
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
