// Per-row (per-token / per-output-channel) and per-tensor quantization of a
// bf16 matrix to OCP e4m3fn or int8 codes, gfx950.
//
// Row kernel: one wavefront per row.  The whole row stays in VGPRs (NV 16-byte
// vectors per lane, 64 lanes read 1 KiB contiguous per step), so X is read from
// HBM exactly once: abs-max over packed bf16 bit patterns (v_pk_max_u16), a
// butterfly wave reduction, one IEEE reciprocal per row, then a 3-op
// correctly rounded quotient per element and 8-byte coalesced code stores.
// Algorithmic traffic: 2*K read + K written + 4 bytes of scale per row.
#include <mutex>

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

// One row into NV 16-byte vectors per lane (zeros past the row's end).
template <int NV>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ x, int64_t ldx, int64_t row, int nvec,
                                         int lane, uint4 (&v)[NV]) {
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int vec = i * 64 + lane;
        v[i] = vec < nvec ? xr[vec] : make_uint4(0, 0, 0, 0);
    }
}

// Tiled output by half blocks through a whole-row LDS image (K % 128 == 0,
// row0 % 16 == 0, K <= 16384).  A workgroup of 8 waves owns 8 rows (half of a
// 16-row block), one row per wave held in VGPRs as in the row kernel above.
// The codes of all 8 rows are written into an LDS image of 8 x K bytes, then
// read back in the order of the tiled layout and stored as 16-byte pieces:
// inside the 2 KiB tile of k-step s, the half block's rows fill four 128-byte
// runs per 1 KiB half (rows 8 * half + r of fragment group q at slot
// 8 * half + r + 16 q), so 64 consecutive threads store 8 whole 128-byte
// lines.  Two barriers per unit: one before the read-back, one before the
// image is written again.
//
// Image: row r at r * W, W = K rounded up to 256 bytes; its 16-byte chunk c
// (codes 16 c .. 16 c + 15) sits at chunk (c & ~15) | ((c & 15) ^ g(r)),
// g(r) = (r & 1) | (r >> 1) << 2, which stays inside the row's W bytes.
// A wave's 8-byte writes (one row, consecutive chunks) stay a permutation of
// 256-byte groups, and the read-back of 16 consecutive slots (rows 0..7 of
// two fragment groups q, q + 1, chunks c and c ^ 2) hits 16 distinct 16-byte
// bank groups.  Each workgroup walks units u, u + grid, ...; the next unit's
// rows are loaded into a second register set before the read-back, so reads
// of X overlap the stores.
__device__ __forceinline__ int img_chunk(int c, int r) { return (c & ~15) | ((c & 15) ^ ((r & 1) | ((r >> 1) << 2))); }

template <int FMT, int ROUND, int NV, bool PREFETCH>
__global__ __launch_bounds__(512) void quant_rows_tiled_img_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                   int64_t units, int k, uint8_t* __restrict__ q,
                                                                   int64_t row0, float* __restrict__ scales) {
    extern __shared__ __attribute__((aligned(16))) uint8_t img[];
    const int lane = threadIdx.x & 63;
    const int r = threadIdx.x >> 6;  // row within the unit
    const int nvec = k >> 3;
    const int64_t steps = k >> 7;
    const int w = (k + 255) & ~255;  // image row stride
    uint4 v[NV], vn[PREFETCH ? NV : 1];
    int64_t u = blockIdx.x;
    if (u < units) load_row<NV>(x, ldx, 8 * u + r, nvec, lane, v);
    while (u < units) {
        const int64_t row = 8 * u + r;
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            m = pk_abs_max(m, v[i].x);
            m = pk_abs_max(m, v[i].y);
            m = pk_abs_max(m, v[i].z);
            m = pk_abs_max(m, v[i].w);
        }
        const float amax = wave_max(amax_from_packed(m));
        RowQuant<FMT, ROUND> rq;
        rq.init(amax);
        if (lane == 0) scales[row] = rq.s;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vec = i * 64 + lane;  // codes 8 vec .. 8 vec + 7: chunk vec / 2, half vec % 2
            if (vec < nvec) {
                uint2 out;
                out.x = rq.pack4(v[i].x, v[i].y);
                out.y = rq.pack4(v[i].z, v[i].w);
                *reinterpret_cast<uint2*>(img + r * w + img_chunk(vec >> 1, r) * 16 + (vec & 1) * 8) = out;
            }
        }
        const int64_t un = u + gridDim.x;
        if constexpr (PREFETCH) {
            if (un < units) load_row<NV>(x, ldx, 8 * un + r, nvec, lane, vn);
        }
        __syncthreads();
        // Read-back: slot t = ((s * 2 + h) * 4 + qq) * 8 + rr holds row rr,
        // codes 128 s + 32 qq + 16 h .. + 15.
        const int64_t blk = (row0 + 8 * u) >> 4;
        const int half = (int)(((row0 + 8 * u) >> 3) & 1);
        uint8_t* const qb = q + blk * steps * 2048;
        const int slots = k >> 1;  // 8 rows x k bytes / 16
        for (int t = threadIdx.x; t < slots; t += 512) {
            const int rr = t & 7, qq = (t >> 3) & 3, h = (t >> 5) & 1, s = t >> 6;
            const int c = 8 * s + 2 * qq + h;
            const uint4 val = *reinterpret_cast<const uint4*>(img + rr * w + img_chunk(c, rr) * 16);
            *reinterpret_cast<uint4*>(qb + (int64_t)s * 2048 + h * 1024 + (8 * half + rr + 16 * qq) * 16) = val;
        }
        __syncthreads();  // the image is written again by the next unit
        if constexpr (PREFETCH) {
#pragma unroll
            for (int i = 0; i < NV; ++i) v[i] = vn[i];
        } else if (un < units) {
            load_row<NV>(x, ldx, 8 * un + r, nvec, lane, v);
        }
        u = un;
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
    for (int64_t j = threadIdx.x; j < k; j += 256) amax = mag_max(amax, fabsf(bf16_lo(xr[j])));
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = mag_max(mag_max(red[0], red[1]), mag_max(red[2], red[3]));
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

template <int FMT, int ROUND, int NV, bool PREFETCH>
static hipError_t launch_rows_tiled_img_cfg(const uint16_t* x, int64_t ldx, int64_t blocks, int64_t k, uint8_t* q,
                                            int64_t row0, float* scales, int per_cu, hipStream_t st) {
    const int64_t units = blocks * 2;
    const int64_t img_bytes = 8 * ((k + 255) & ~int64_t(255));
    const int64_t cap = 256 * (int64_t)per_cu;
    const int64_t grid = units < cap ? units : cap;
    // Images above 64 KiB (K > 8192) need the kernel's dynamic LDS limit raised.
    static const hipError_t lds_limit = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&quant_rows_tiled_img_kernel<FMT, ROUND, NV, PREFETCH>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 8 * ((512 * NV + 255) & ~255));
    if (lds_limit != hipSuccess) return lds_limit;
    hipLaunchKernelGGL((quant_rows_tiled_img_kernel<FMT, ROUND, NV, PREFETCH>), dim3((unsigned)grid), dim3(512),
                       (size_t)img_bytes, st, x, ldx, units, (int)k, q, row0, scales);
    return hipGetLastError();
}

template <int FMT, int ROUND, int NV>
static hipError_t launch_rows_tiled_img(const uint16_t* x, int64_t ldx, int64_t blocks, int64_t k, uint8_t* q,
                                        int64_t row0, float* scales, hipStream_t st) {
    // Workgroups of 8 waves: two per CU while the image (8 W bytes) and two
    // row register sets per lane (128 VGPRs) fit twice, else one.
    const int64_t img_bytes = 8 * ((k + 255) & ~int64_t(255));
    const int per_cu = (NV <= 12 && img_bytes <= 80 * 1024) ? 2 : 1;
    return launch_rows_tiled_img_cfg<FMT, ROUND, NV, true>(x, ldx, blocks, k, q, row0, scales, per_cu, st);
}

template <int FMT, int ROUND>
static hipError_t dispatch_rows_tiled_img(const uint16_t* x, int64_t ldx, int64_t blocks, int64_t k, uint8_t* q,
                                            int64_t row0, float* scales, hipStream_t st) {
    const int64_t nv = (k + 511) / 512;
    if (nv <= 2) return launch_rows_tiled_img<FMT, ROUND, 2>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 4) return launch_rows_tiled_img<FMT, ROUND, 4>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 8) return launch_rows_tiled_img<FMT, ROUND, 8>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 10) return launch_rows_tiled_img<FMT, ROUND, 10>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 11) return launch_rows_tiled_img<FMT, ROUND, 11>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 14) return launch_rows_tiled_img<FMT, ROUND, 14>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 16) return launch_rows_tiled_img<FMT, ROUND, 16>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 24) return launch_rows_tiled_img<FMT, ROUND, 24>(x, ldx, blocks, k, q, row0, scales, st);
    if (nv <= 28) return launch_rows_tiled_img<FMT, ROUND, 28>(x, ldx, blocks, k, q, row0, scales, st);
    return launch_rows_tiled_img<FMT, ROUND, 32>(x, ldx, blocks, k, q, row0, scales, st);
}

template <int FMT, int ROUND, bool TILED>
static hipError_t dispatch_rows(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, uint8_t* q, int64_t ldq,
                                int64_t row0, float* scales, hipStream_t st) {
    const bool aligned = (k % 8 == 0) && (ldx % 8 == 0) && (TILED || ldq % 8 == 0) &&
                         ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
    const int64_t nv = (k + 511) / 512;
    // Tiled output from a block boundary: whole 16-row blocks by the image
    // kernel (16-byte aligned codes), the remaining rows below.
    if constexpr (TILED) {
        if (aligned && nv <= 32 && row0 % 16 == 0 && rows >= 16 && (uintptr_t)q % 16 == 0) {
            const int64_t blocks = rows / 16;
            hipError_t e = dispatch_rows_tiled_img<FMT, ROUND>(x, ldx, blocks, k, q, row0, scales, st);
            if (e != hipSuccess || rows == 16 * blocks) return e;
            x += 16 * blocks * ldx;
            scales += 16 * blocks;
            row0 += 16 * blocks;
            rows -= 16 * blocks;
        }
    }
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

// One element of the per-tensor quantizer: e4m3(clamp(bf16(x / s), +-448)),
// with x / s the correctly rounded binary32 quotient for any divisor.
struct TensorQuant {
    float s, r;
    __device__ __forceinline__ float quotient(float f) const { return div_rn_any(f, s, r); }
    // Two bf16 -> two codes: binary32 quotients, rounded to bf16 together
    // (v_cvt_pk_bf16_f32, round to nearest even), clamped, converted.
    __device__ __forceinline__ uint32_t pack2(uint32_t w) const {
        const uint32_t b = pack_bf16x2(quotient(bf16_lo(w)), quotient(bf16_hi(w)));
        return cvt_e4m3x2(clamp_e4m3(bf16_lo(b)), clamp_e4m3(bf16_hi(b)));
    }
    __device__ __forceinline__ uint32_t pack4(uint32_t w0, uint32_t w1) const { return pack2(w0) | (pack2(w1) << 16); }
    // The codes of one 16-byte vector (8 bf16), as pack4 twice, with one test
    // per vector in place of a branch per element: the quotients by the three
    // operations of div_rn_any (the quotient of a zero kept as q0 = x * r, so
    // its sign follows a negative static scale as IEEE division does), and if
    // any of them is not finite (an infinity or NaN in x; a zero, infinite or
    // NaN scale; an overflowing quotient or reciprocal) the vector is redone
    // by pack4, whose quotients fall back to IEEE division and whose clamp
    // keeps a NaN.  A finite quotient needs neither, so the common path clamps
    // with v_med3 alone.
    __device__ __forceinline__ uint2 pack8(const uint4& v) const {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        float q[8];
        bool bad = false;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float f = (j & 1) ? bf16_hi(w[j >> 1]) : bf16_lo(w[j >> 1]);
            const float q0 = f * r;
            const float q1 = fmaf(fmaf(-q0, s, f), r, q0);
            bad |= !__builtin_isfinite(q1);
            q[j] = f == 0.0f ? q0 : q1;
        }
        if (bad) return make_uint2(pack4(v.x, v.y), pack4(v.z, v.w));
        uint32_t c[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = pack_bf16x2(q[2 * j], q[2 * j + 1]);
            c[j] = cvt_e4m3x2(__builtin_amdgcn_fmed3f(bf16_lo(b), -kE4M3Max, kE4M3Max),
                              __builtin_amdgcn_fmed3f(bf16_hi(b), -kE4M3Max, kE4M3Max));
        }
        return make_uint2(c[0] | (c[1] << 16), c[2] | (c[3] << 16));
    }
};

// Maximum of a workgroup's per-wave magnitudes (NaN kept), on every thread.
__device__ __forceinline__ float block_max4(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return mag_max(mag_max(red[0], red[1]), mag_max(red[2], red[3]));
}

// Scale of pass 2: the static scale, or the fold of the partial maxima
// (at most 1024: four loads per thread, issued together).
__device__ __forceinline__ TensorQuant tensor_scale(const float* __restrict__ partial, int nparts,
                                                    const float* __restrict__ static_scale, int bf16_divisor,
                                                    float* red, float* __restrict__ scale_out) {
    TensorQuant tq;
    if (static_scale) {
        tq.s = *static_scale;
    } else {
        float p[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = (int)threadIdx.x + 256 * k;
            p[k] = partial[i < nparts ? i : nparts - 1];
        }
        const float a = block_max4(mag_max(mag_max(p[0], p[1]), mag_max(p[2], p[3])), red);
        tq.s = amax_scale(a, kE4M3Recip);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = tq.s;
    if (bf16_divisor) tq.s = round_to_bf16(tq.s);
    tq.r = 1.0f / tq.s;
    return tq;
}

// Vector path (K % 8 == 0, 16-byte aligned rows, K <= NV * 512): one wave per
// row, NV 16-byte loads per lane issued together.  Lanes past the row re-read
// its last vector (harmless for a maximum; their codes are not stored).
template <int NV>
__global__ __launch_bounds__(256) void tensor_amax_vec_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                              int64_t rows, int k, float* __restrict__ partial) {
    __shared__ float red[4];
    const int lane = threadIdx.x & 63;
    const int nvec = k >> 3;
    int off[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) off[i] = (i * 64 + lane < nvec ? i * 64 + lane : nvec - 1) * 8;
    uint32_t m = 0;
    const int64_t step = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += step) {
        const uint16_t* xr = x + row * ldx;
        uint4 v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = *reinterpret_cast<const uint4*>(xr + off[i]);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            m = pk_abs_max(m, v[i].x);
            m = pk_abs_max(m, v[i].y);
            m = pk_abs_max(m, v[i].z);
            m = pk_abs_max(m, v[i].w);
        }
    }
    const float a = block_max4(amax_from_packed(m), red);
    if (threadIdx.x == 0) partial[blockIdx.x] = a;
}

// bf16_divisor: divide by bf16(s) (IEEE) instead of s, keeping s as the
// returned scale.
template <int NV>
__global__ __launch_bounds__(256) void tensor_quant_vec_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                               int64_t rows, int k, const float* __restrict__ partial,
                                                               int nparts, const float* __restrict__ static_scale,
                                                               int bf16_divisor, uint8_t* __restrict__ q,
                                                               int64_t ldq, float* __restrict__ scale_out) {
    __shared__ float red[4];
    const TensorQuant tq = tensor_scale(partial, nparts, static_scale, bf16_divisor, red, scale_out);
    const int lane = threadIdx.x & 63;
    const int nvec = k >> 3;
    int off[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) off[i] = (i * 64 + lane < nvec ? i * 64 + lane : nvec - 1) * 8;
    const int64_t step = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += step) {
        const uint16_t* xr = x + row * ldx;
        uint8_t* qr = q + row * ldq;
        uint4 v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = *reinterpret_cast<const uint4*>(xr + off[i]);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (i * 64 + lane < nvec) *reinterpret_cast<uint2*>(qr + off[i]) = tq.pack8(v[i]);
        }
    }
}

// General path (any K and alignment): elementwise, a band of rows per workgroup.
__global__ __launch_bounds__(256) void tensor_amax_any_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                              int64_t rows, int64_t k, int64_t rows_per_block,
                                                              float* __restrict__ partial) {
    __shared__ float red[4];
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    float amax = 0.0f;
    for (int64_t r = r0; r < r1; ++r)
        for (int64_t j = threadIdx.x; j < k; j += 256) amax = mag_max(amax, fabsf(bf16_lo(x[r * ldx + j])));
    const float a = block_max4(amax, red);
    if (threadIdx.x == 0) partial[blockIdx.x] = a;
}

__global__ __launch_bounds__(256) void tensor_quant_any_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                               int64_t rows, int64_t k, int64_t rows_per_block,
                                                               const float* __restrict__ partial, int nparts,
                                                               const float* __restrict__ static_scale,
                                                               int bf16_divisor, uint8_t* __restrict__ q,
                                                               int64_t ldq, float* __restrict__ scale_out) {
    __shared__ float red[4];
    const TensorQuant tq = tensor_scale(partial, nparts, static_scale, bf16_divisor, red, scale_out);
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    for (int64_t r = r0; r < r1; ++r)
        for (int64_t j = threadIdx.x; j < k; j += 256) q[r * ldq + j] = (uint8_t)(tq.pack2(x[r * ldx + j]) & 0xFFu);
}

// Typed general path: bf16, fp16 or fp32 input, elementwise, a band of rows
// per workgroup.  The quotient follows one of the reference's two forms:
//   eager  (torch's clamp(x / s, +-448) in x's dtype, FL/inference/
//          fused_kernels.py:773 and fp8.py:107-113): divisor and quotient
//          rounded to x's dtype (bf16 or fp16; nothing for fp32),
//   triton (FL/inference/fused_kernels.py:240-246): fp32 divisor, quotient
//          rounded to bf16, whatever x's dtype.
// A NaN quotient (0 / 0 when an fp16 divisor underflows to zero) stays NaN
// through the clamp, as torch.clamp keeps it, and becomes 0x7F, the float8
// cast of the device's canonical (positive) NaN.
template <int IN>
__device__ __forceinline__ float load_in(const void* __restrict__ x, int64_t i) {
    if constexpr (IN == kInBF16) return __uint_as_float((uint32_t)((const uint16_t*)x)[i] << 16);
    else if constexpr (IN == kInF16) return (float)((const _Float16*)x)[i];
    else return ((const float*)x)[i];
}

template <int IN>
__global__ __launch_bounds__(256) void tensor_amax_typed_kernel(const void* __restrict__ x, int64_t ldx, int64_t rows,
                                                                int64_t k, int64_t rows_per_block,
                                                                float* __restrict__ partial) {
    __shared__ float red[4];
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    float amax = 0.0f;
    for (int64_t r = r0; r < r1; ++r)
        for (int64_t j = threadIdx.x; j < k; j += 256) amax = mag_max(amax, fabsf(load_in<IN>(x, r * ldx + j)));
    const float a = block_max4(amax, red);
    if (threadIdx.x == 0) partial[blockIdx.x] = a;
}

template <int IN>
__global__ __launch_bounds__(256) void tensor_quant_typed_kernel(const void* __restrict__ x, int64_t ldx, int64_t rows,
                                                                 int64_t k, int64_t rows_per_block,
                                                                 const float* __restrict__ partial, int nparts,
                                                                 const float* __restrict__ static_scale, int eager,
                                                                 uint8_t* __restrict__ q, int64_t ldq,
                                                                 float* __restrict__ scale_out) {
    __shared__ float red[4];
    TensorQuant tq = tensor_scale(partial, nparts, static_scale, 0, red, scale_out);
    // Rounding of divisor and quotient: 0 none, 1 bf16, 2 fp16.
    const int rnd = !eager ? 1 : IN == kInBF16 ? 1 : IN == kInF16 ? 2 : 0;
    if (eager && rnd == 1) tq.s = round_to_bf16(tq.s);
    if (eager && rnd == 2) tq.s = (float)(_Float16)tq.s;
    tq.r = 1.0f / tq.s;
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t j = threadIdx.x; j < k; j += 256) {
            float v = tq.quotient(load_in<IN>(x, r * ldx + j));
            if (rnd == 1) v = round_to_bf16(v);
            if (rnd == 2) v = (float)(_Float16)v;
            uint32_t code;
            if (v != v) code = 0x7Fu;
            else code = cvt_e4m3x2(clamp_e4m3(v), 0.0f) & 0xFFu;
            q[r * ldq + j] = (uint8_t)code;
        }
    }
}

namespace {

constexpr int64_t kTensorBlocks = 1024;

int64_t tensor_blocks(int64_t rows) { return (rows + 3) / 4 < kTensorBlocks ? (rows + 3) / 4 : kTensorBlocks; }

bool tensor_vec(const uint16_t* x, int64_t ldx, int64_t k, const uint8_t* q, int64_t ldq) {
    return k % 8 == 0 && ldx % 8 == 0 && ldq % 8 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)q % 8 == 0 &&
           (k + 511) / 512 <= 32;
}

template <int NV>
hipError_t launch_tensor_vec(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, const float* static_scale,
                             bool bf16_divisor, float* partial, uint8_t* q, int64_t ldq, float* scale_out,
                             hipStream_t st) {
    const int64_t blocks = tensor_blocks(rows);
    if (!static_scale) {
        hipLaunchKernelGGL((tensor_amax_vec_kernel<NV>), dim3((unsigned)blocks), dim3(256), 0, st, x, ldx, rows,
                           (int)k, partial);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((tensor_quant_vec_kernel<NV>), dim3((unsigned)blocks), dim3(256), 0, st, x, ldx, rows, (int)k,
                       (const float*)partial, (int)blocks, static_scale, (int)bf16_divisor, q, ldq, scale_out);
    return hipGetLastError();
}

}  // namespace

// Partial maxima written by pass 1: one per workgroup of either path.
int64_t tensor_quant_parts(int64_t rows, int64_t k) {
    (void)k;
    return rows < 1 ? 1 : (rows < kTensorBlocks ? rows : kTensorBlocks);
}

// Scratch of the allocation-free per-tensor quantizer: room for the partial
// maxima of any call (at most kTensorBlocks).  Every block of pass 1 writes
// its own entry before pass 2 reads it, so nothing needs clearing between
// calls; two calls that overlap on one GPU share it and race.  Each device
// holds its own copy; host code must use the device address from
// tensor_scratch(), never the symbol itself.
static __device__ __align__(256) float scratch[kTensorScratchFloats];
static_assert(kTensorScratchFloats >= kTensorBlocks, "scratch holds every partial maximum");

hipError_t tensor_scratch(float** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex lock;
    static float* addresses[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(lock);
    if (!addresses[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));  // the current device's copy
        if (e != hipSuccess) return e;
        addresses[dev] = (float*)ptr;
    }
    *out = addresses[dev];
    return hipSuccess;
}

hipError_t launch_quant_tensor_e4m3(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k,
                                    const float* static_scale, bool bf16_divisor, float* partial, uint8_t* q,
                                    int64_t ldq, float* scale_out, hipStream_t st) {
    if (tensor_vec(x, ldx, k, q, ldq)) {
        const int64_t nv = (k + 511) / 512;
        if (nv <= 2) return launch_tensor_vec<2>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 4) return launch_tensor_vec<4>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 8) return launch_tensor_vec<8>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 10) return launch_tensor_vec<10>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 11) return launch_tensor_vec<11>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 14) return launch_tensor_vec<14>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 16) return launch_tensor_vec<16>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 24) return launch_tensor_vec<24>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        if (nv <= 28) return launch_tensor_vec<28>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
        return launch_tensor_vec<32>(x, ldx, rows, k, static_scale, bf16_divisor, partial, q, ldq, scale_out, st);
    }
    // Bands of rows: at most 1024 workgroups (the fold reads one partial each).
    const int64_t blocks = rows < kTensorBlocks ? rows : kTensorBlocks;
    const int64_t rpb = (rows + blocks - 1) / blocks;
    const int64_t used = (rows + rpb - 1) / rpb;
    if (!static_scale) {
        hipLaunchKernelGGL(tensor_amax_any_kernel, dim3((unsigned)used), dim3(256), 0, st, x, ldx, rows, k, rpb,
                           partial);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(tensor_quant_any_kernel, dim3((unsigned)used), dim3(256), 0, st, x, ldx, rows, k, rpb,
                       (const float*)partial, (int)used, static_scale, (int)bf16_divisor, q, ldq, scale_out);
    return hipGetLastError();
}

hipError_t launch_quant_tensor_e4m3_typed(const void* x, int in, bool eager, int64_t ldx, int64_t rows, int64_t k,
                                          const float* static_scale, float* partial, uint8_t* q, int64_t ldq,
                                          float* scale_out, hipStream_t st) {
    if (in == kInBF16)
        return launch_quant_tensor_e4m3((const uint16_t*)x, ldx, rows, k, static_scale, eager, partial, q, ldq,
                                        scale_out, st);
    const int64_t blocks = rows < kTensorBlocks ? rows : kTensorBlocks;
    const int64_t rpb = (rows + blocks - 1) / blocks;
    const int64_t used = (rows + rpb - 1) / rpb;
    if (!static_scale) {
        if (in == kInF16)
            hipLaunchKernelGGL(tensor_amax_typed_kernel<kInF16>, dim3((unsigned)used), dim3(256), 0, st, x, ldx, rows,
                               k, rpb, partial);
        else
            hipLaunchKernelGGL(tensor_amax_typed_kernel<kInF32>, dim3((unsigned)used), dim3(256), 0, st, x, ldx, rows,
                               k, rpb, partial);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (in == kInF16)
        hipLaunchKernelGGL(tensor_quant_typed_kernel<kInF16>, dim3((unsigned)used), dim3(256), 0, st, x, ldx, rows, k,
                           rpb, (const float*)partial, (int)used, static_scale, (int)eager, q, ldq, scale_out);
    else
        hipLaunchKernelGGL(tensor_quant_typed_kernel<kInF32>, dim3((unsigned)used), dim3(256), 0, st, x, ldx, rows, k,
                           rpb, (const float*)partial, (int)used, static_scale, (int)eager, q, ldq, scale_out);
    return hipGetLastError();
}

}  // namespace h3q
