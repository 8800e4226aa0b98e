// Per-row (per-token / per-output-channel) and per-tensor quantization of a
// bf16 matrix to OCP e4m3fn or int8 codes, gfx950.
//
// Row kernel: one wavefront per row.  The whole row stays in VGPRs (NV 16-byte
// vectors per lane, 64 lanes read 1 KiB contiguous per step), so X is read from
// HBM exactly once: abs-max over packed bf16 bit patterns (v_pk_max_u16), a
// butterfly wave reduction, one IEEE reciprocal per row, then a 3-op
// correctly rounded quotient per element and 8-byte coalesced code stores.
// Algorithmic traffic: 2*K read + K written + 4 bytes of scale per row.
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"
#include "row_quant.hpp"

namespace h3q {

// Byte offset of code (row, k) in the output.  Row-major: row * ldq + k.
// Tiled (the weight layout of the GEMMs, K % 128 == 0, ldq = K / 128 steps):
// 16-row x 128-byte blocks of 2 KiB, block (row / 16, k / 128) at
// ((row / 16) * steps + k / 128) * 2048; inside it byte k % 128 of row r lands
// at (k % 32 / 16) * 1024 + (r % 16 + 16 * (k % 128 / 32)) * 16 + k % 16.
// That is the operand order of v_mfma_*_16x16x128: lane l = r % 16 +
// 16 * (k % 128 / 32) holds bytes k % 32 of its 32-byte fragment, in two
// 16-byte halves 1 KiB apart.
template <bool TILED>
__device__ __forceinline__ int64_t code_offset(int64_t row, int64_t k, int64_t ldq) {
    if constexpr (!TILED) return row * ldq + k;
    const int64_t kk = k & 127;
    const int64_t lane = (row & 15) + 16 * (kk >> 5);
    return (((row >> 4) * ldq + (k >> 7)) << 11) + (((kk >> 4) & 1) << 10) + (lane << 4) + (kk & 15);
}

// Vector path: K % 8 == 0, x rows 16-byte aligned, q rows 8-byte aligned, K <= NV*512.
// TILED: codes go to the tiled layout at absolute row row0 + row.
template <int FMT, int ROUND, int NV, bool TILED>
__global__ __launch_bounds__(256) void quant_rows_vec_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             int64_t rows, int k, uint8_t* __restrict__ q,
                                                             int64_t ldq, int64_t row0,
                                                             float* __restrict__ scales) {
    const int lane = threadIdx.x & 63;
    const int nvec = k >> 3;
    // Rows are dealt to waves in order (row = wave id + i * waves in the grid),
    // so the rows in flight at any moment form one contiguous band of X.
    const int64_t step = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += step) {
        const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
        uint4 v[NV];
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vec = i * 64 + lane;
            if (vec < nvec) {
                v[i] = xr[vec];
            } else {
                v[i] = make_uint4(0, 0, 0, 0);
            }
            m = pk_abs_max(m, v[i].x);
            m = pk_abs_max(m, v[i].y);
            m = pk_abs_max(m, v[i].z);
            m = pk_abs_max(m, v[i].w);
        }
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
                *reinterpret_cast<uint2*>(q + code_offset<TILED>(row0 + row, 8 * (int64_t)vec, ldq)) = out;
            }
        }
        if (lane == 0) scales[row] = rq.s;
    }
}

// General path (any K, any alignment): one workgroup per row, two passes.
template <int FMT, int ROUND, bool TILED>
__global__ __launch_bounds__(256) void quant_rows_any_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             int64_t rows, int64_t k, uint8_t* __restrict__ q,
                                                             int64_t ldq, int64_t row0,
                                                             float* __restrict__ scales) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * ldx;
    float amax = 0.0f;
    for (int64_t j = threadIdx.x; j < k; j += 256) amax = fmaxf(amax, fabsf(bf16_lo(xr[j])));
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    RowQuant<FMT, ROUND> rq;
    rq.init(amax);
    for (int64_t j = threadIdx.x; j < k; j += 256) {
        uint32_t w = xr[j];
        q[code_offset<TILED>(row0 + row, j, ldq)] = (uint8_t)(rq.pack4(w, 0u) & 0xFFu);
    }
    if (threadIdx.x == 0) scales[row] = rq.s;
}

constexpr int64_t kRowBlocks = 1024;

template <int FMT, int ROUND, int NV, bool TILED>
static hipError_t launch_rows_vec(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, uint8_t* q,
                                  int64_t ldq, int64_t row0, float* scales, hipStream_t st) {
    // One wave per row up to 4 waves per SIMD of the chip (1024 workgroups of
    // four waves on 256 CUs); beyond that each wave takes several rows.
    const int64_t blocks = (rows + 3) / 4 < kRowBlocks ? (rows + 3) / 4 : kRowBlocks;
    hipLaunchKernelGGL((quant_rows_vec_kernel<FMT, ROUND, NV, TILED>), dim3((unsigned)blocks), dim3(256), 0, st, x,
                       ldx, rows, (int)k, q, ldq, row0, scales);
    return hipGetLastError();
}

template <int FMT, int ROUND, bool TILED>
static hipError_t dispatch_rows(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, uint8_t* q, int64_t ldq,
                                int64_t row0, float* scales, hipStream_t st) {
    const bool aligned = (k % 8 == 0) && (ldx % 8 == 0) && (TILED || ldq % 8 == 0) &&
                         ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
    const int64_t nv = (k + 511) / 512;
    if (aligned) {
        if (nv <= 2) return launch_rows_vec<FMT, ROUND, 2, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 4) return launch_rows_vec<FMT, ROUND, 4, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        // nv = 16-byte vectors per lane (512 columns each); exact sizes for the H3
        // and benchmark widths (K = 5120, 5376, 7168, 13824) keep no idle vectors.
        if (nv <= 8) return launch_rows_vec<FMT, ROUND, 8, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 10) return launch_rows_vec<FMT, ROUND, 10, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 11) return launch_rows_vec<FMT, ROUND, 11, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 14) return launch_rows_vec<FMT, ROUND, 14, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 16) return launch_rows_vec<FMT, ROUND, 16, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 24) return launch_rows_vec<FMT, ROUND, 24, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 28) return launch_rows_vec<FMT, ROUND, 28, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
        if (nv <= 32) return launch_rows_vec<FMT, ROUND, 32, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
    }
    hipLaunchKernelGGL((quant_rows_any_kernel<FMT, ROUND, TILED>), dim3((unsigned)rows), dim3(256), 0, st, x, ldx,
                       rows, k, q, ldq, row0, scales);
    return hipGetLastError();
}

template <bool TILED>
static hipError_t launch_quant_rows_layout(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, int fmt,
                                           int rounding, uint8_t* q, int64_t ldq, int64_t row0, float* scales,
                                           hipStream_t st) {
    if (fmt == kFmtE4M3) return dispatch_rows<kFmtE4M3, kRoundDiv, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
    if (rounding == kRoundDiv)
        return dispatch_rows<kFmtInt8, kRoundDiv, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
    return dispatch_rows<kFmtInt8, kRoundRcpMul, TILED>(x, ldx, rows, k, q, ldq, row0, scales, st);
}

hipError_t launch_quant_rows(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, int fmt, int rounding,
                             uint8_t* q, int64_t ldq, float* scales, hipStream_t st) {
    return launch_quant_rows_layout<false>(x, ldx, rows, k, fmt, rounding, q, ldq, 0, scales, st);
}

hipError_t launch_quant_rows_tiled(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, int fmt, int rounding,
                                   uint8_t* q_tiled, int64_t row0, float* scales, hipStream_t st) {
    return launch_quant_rows_layout<true>(x, ldx, rows, k, fmt, rounding, q_tiled, k / 128, row0, scales, st);
}

// ---------------------------------------------------------------- per-tensor

// Pass 1: each workgroup reduces |x| over a contiguous band of rows.
__global__ __launch_bounds__(256) void tensor_amax_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
                                                          int64_t k, int64_t rows_per_block,
                                                          float* __restrict__ partial) {
    __shared__ float red[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    const bool vec = (k % 8 == 0) && (ldx % 8 == 0) && ((uintptr_t)x % 16 == 0);
    uint32_t m = 0;
    float amax = 0.0f;
    for (int64_t r = r0 + wave; r < r1; r += 4) {
        const uint16_t* xr = x + r * ldx;
        if (vec) {
            const uint4* xv = reinterpret_cast<const uint4*>(xr);
            for (int64_t j = lane; j < (k >> 3); j += 64) {
                uint4 v = xv[j];
                m = pk_abs_max(m, v.x);
                m = pk_abs_max(m, v.y);
                m = pk_abs_max(m, v.z);
                m = pk_abs_max(m, v.w);
            }
        } else {
            for (int64_t j = lane; j < k; j += 64) amax = fmaxf(amax, fabsf(bf16_lo(xr[j])));
        }
    }
    amax = wave_max(fmaxf(amax, amax_from_packed(m)));
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One element of the per-tensor quantizer: e4m3(clamp(bf16(x / s), +-448)).
struct TensorQuant {
    float s, r;
    bool exact_div;  // static scale or bf16 divisor: IEEE division
    __device__ __forceinline__ float value(float f) const {
        float qv = exact_div ? __fdiv_rn(f, s) : copysignf(div_rn(f, s, r), f);
        return __builtin_amdgcn_fmed3f(round_to_bf16(qv), -kE4M3Max, kE4M3Max);
    }
    __device__ __forceinline__ uint32_t pack4(uint32_t w0, uint32_t w1) const {
        return cvt_e4m3x2(value(bf16_lo(w0)), value(bf16_hi(w0))) |
               (cvt_e4m3x2(value(bf16_lo(w1)), value(bf16_hi(w1))) << 16);
    }
};

// Pass 2: every workgroup folds the partial maxima (or reads the static
// scale), then quantizes its band of rows.
// bf16_divisor: divide by bf16(s) (IEEE) instead of s, keeping s as the
// returned scale.
__global__ __launch_bounds__(256) void tensor_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           int64_t rows, int64_t k, int64_t rows_per_block,
                                                           const float* __restrict__ partial, int nparts,
                                                           const float* __restrict__ static_scale,
                                                           int bf16_divisor, uint8_t* __restrict__ q,
                                                           int64_t ldq, float* __restrict__ scale_out) {
    __shared__ float red[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    TensorQuant tq;
    if (static_scale) {
        tq.s = *static_scale;
        tq.exact_div = true;
    } else {
        float a = 0.0f;
        for (int i = threadIdx.x; i < nparts; i += 256) a = fmaxf(a, partial[i]);
        a = wave_max(a);
        if (lane == 0) red[wave] = a;
        __syncthreads();
        a = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        tq.s = amax_scale(a, kE4M3Recip);
        tq.exact_div = false;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = tq.s;
    if (bf16_divisor) {
        tq.s = round_to_bf16(tq.s);
        tq.exact_div = true;
    }
    tq.r = 1.0f / tq.s;
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    const bool vec = (k % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && ((uintptr_t)x % 16 == 0) &&
                     ((uintptr_t)q % 8 == 0);
    for (int64_t r = r0 + wave; r < r1; r += 4) {
        const uint16_t* xr = x + r * ldx;
        uint8_t* qr = q + r * ldq;
        if (vec) {
            const uint4* xv = reinterpret_cast<const uint4*>(xr);
            uint2* qv = reinterpret_cast<uint2*>(qr);
            for (int64_t j = lane; j < (k >> 3); j += 64) {
                uint4 v = xv[j];
                uint2 o;
                o.x = tq.pack4(v.x, v.y);
                o.y = tq.pack4(v.z, v.w);
                qv[j] = o;
            }
        } else {
            for (int64_t j = lane; j < k; j += 64) qr[j] = (uint8_t)(tq.pack4(xr[j], 0u) & 0xFFu);
        }
    }
}

int64_t tensor_quant_parts(int64_t rows, int64_t k) {
    // Enough bands to fill the chip for the amax pass, few enough that every
    // workgroup of the second pass folds them quickly.
    const int64_t elems = rows * k;
    int64_t parts = (elems + 65535) / 65536;
    if (parts > 1024) parts = 1024;
    if (parts > rows) parts = rows;
    return parts < 1 ? 1 : parts;
}

hipError_t launch_quant_tensor_e4m3(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k,
                                    const float* static_scale, bool bf16_divisor, float* partial, uint8_t* q,
                                    int64_t ldq, float* scale_out, hipStream_t st) {
    const int64_t parts = tensor_quant_parts(rows, k);
    const int64_t rpb = (rows + parts - 1) / parts;
    const int64_t blocks = (rows + rpb - 1) / rpb;
    if (!static_scale) {
        hipLaunchKernelGGL(tensor_amax_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, ldx, rows, k, rpb,
                           partial);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(tensor_quant_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, ldx, rows, k, rpb,
                       (const float*)partial, (int)blocks, static_scale, (int)bf16_divisor, q, ldq, scale_out);
    return hipGetLastError();
}

}  // namespace h3q
