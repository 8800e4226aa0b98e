// Per-(batch, head) FP8 quantization of attention operands, gfx950: the
// reference's quantize_fp8_e4m3_per_head (FL/inference/fused_kernels.py:823-877,
// Triton kernels :175-227 and :250-273).  For value [B, S, H, D] bf16,
// contiguous:
//
//   scale[b, h] = max(RN(amax_{s,d} |value[b, s, h, d]| * RN(1/448)), 1e-12)
//   q[b, s, h, d] = e4m3fn(clamp(value / scale[b, h], +-448))
//
// with the quotient a correctly rounded binary32 division (bf16 divided by a
// dimensioned fp32 tensor promotes to fp32, no bf16 intermediate) and the
// e4m3fn cast round-to-nearest-even.
//
// A scale needs every token of its (batch, head), so the input is read twice
// (unless it stays in the caches between the launches).  Three launches:
//
//   head_amax_kernel   workgroup (b, chunk g of tokens, column group c), one
//                      wavefront per token row: lane l reads positions
//                      c * 64 NS + l + 64 i, i < NS, of the row (a position is
//                      8 bf16, one 16-byte load; a row's loads are issued
//                      together) and keeps one packed maximum per position;
//                      at the end an LDS max per head and partial[b, h, g, c].
//   head_scale_kernel  one wavefront per (b, h): max over the G * C partials,
//                      scale[b, h].
//   head_quant_kernel  workgroup (b, g, c), one wavefront per row: lane l
//                      quantizes the same positions with the scales of their
//                      heads, read once per wavefront.
//
// A row is split into C column groups of at most 8 positions per lane so
// that a wavefront needs few registers and many wavefronts share a SIMD:
// their loads and their arithmetic then overlap.  Traffic per element: 2
// bytes (pass 1) + 2 + 1 bytes (pass 3); algorithmic 3 bytes.
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"
#include "row_quant.hpp"  // pk_abs_max, amax_from_packed

namespace h3q {

namespace {

struct HeadQuantShape {
    int64_t batch, seq, heads, head_dim;
    int64_t chunks;  // G: token chunks per batch of passes 1 and 3
    int64_t rpc;     // tokens per chunk
    int64_t groups;  // C: column groups per row (NS positions per lane each)
};

// Loads and stores of one position: 8 elements as one 16-byte load (IoVec),
// 8 elements one by one (IoVecUnaligned, for a misaligned x or codes), or a
// single element (IoElem, head_dim % 8 != 0).
struct IoVec {
    static constexpr int VEC = 8;
    using T = uint4;
    static __device__ __forceinline__ T load(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
    static __device__ __forceinline__ uint32_t amax_bits(uint32_t m, const T& v) {
        m = pk_abs_max(m, v.x);
        m = pk_abs_max(m, v.y);
        m = pk_abs_max(m, v.z);
        return pk_abs_max(m, v.w);
    }
    template <class Q>
    static __device__ __forceinline__ void store(uint8_t* q, const T& v, const Q& rq) {
        uint2 o;
        o.x = rq.pack4(v.x, v.y);
        o.y = rq.pack4(v.z, v.w);
        *reinterpret_cast<uint2*>(q) = o;
    }
};

struct IoVecUnaligned {
    static constexpr int VEC = 8;
    using T = uint4;
    static __device__ __forceinline__ T load(const uint16_t* p) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = (uint32_t)p[2 * j] | ((uint32_t)p[2 * j + 1] << 16);
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
    static __device__ __forceinline__ uint32_t amax_bits(uint32_t m, const T& v) { return IoVec::amax_bits(m, v); }
    template <class Q>
    static __device__ __forceinline__ void store(uint8_t* q, const T& v, const Q& rq) {
        const uint32_t lo = rq.pack4(v.x, v.y), hi = rq.pack4(v.z, v.w);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            q[j] = (uint8_t)(lo >> (8 * j));
            q[4 + j] = (uint8_t)(hi >> (8 * j));
        }
    }
};

struct IoElem {
    static constexpr int VEC = 1;
    using T = uint32_t;
    static __device__ __forceinline__ T load(const uint16_t* p) { return (uint32_t)*p; }
    static __device__ __forceinline__ uint32_t amax_bits(uint32_t m, const T& v) { return pk_abs_max(m, v); }
    template <class Q>
    static __device__ __forceinline__ void store(uint8_t* q, const T& v, const Q& rq) {
        *q = (uint8_t)(rq.pack4(v, 0u) & 0xFFu);
    }
};

// One position's quantizer: e4m3(x / s) with the correctly rounded binary32
// quotient (div_rn_signed, r = RN(1/s)).  No clamp: |x| <= amax and s = RN(amax *
// RN(1/448)) give |x / s| <= 448 (1 + 2^-22), which v_cvt_pk_fp8_f32 rounds
// to 448 (it saturates everything up to 464; measured on MI355X); a NaN
// quotient stays NaN, as torch's clamp leaves it.
struct HeadQuant {
    float r, dv;  // RN(1/s) and the divisor of the residual correction
    // A head holding an infinity has s = inf and r = 0, where the residual
    // q0 * s - x would be 0 * inf = NaN although x / s is +-0; dividing by 0
    // there leaves q0 = x * 0: +-0 for a finite x, NaN for an infinite one,
    // the IEEE quotients.  For a finite s, dv = s.
    __device__ __forceinline__ void set(float s) {
        r = 1.0f / s;
        dv = s <= 3.402823466e38f ? s : 0.0f;
    }
    __device__ __forceinline__ float value(float f) const { return div_rn_signed(f, dv, r); }
    __device__ __forceinline__ uint32_t pack4(uint32_t w0, uint32_t w1) const {
        return cvt_e4m3x2(value(bf16_lo(w0)), value(bf16_hi(w0))) |
               (cvt_e4m3x2(value(bf16_lo(w1)), value(bf16_hi(w1))) << 16);
    }
};

}  // namespace

// Pass 1.  blockIdx.x = (b * G + g) * C + c.  Dynamic LDS: H words, the
// per-head maxima as bit patterns (non-negative binary32 values order like
// their bits); every head's entry is written, 0 for heads outside group c.
template <class IO, int NS>
__global__ __launch_bounds__(256) void head_amax_kernel(const uint16_t* __restrict__ x, HeadQuantShape sh,
                                                        float* __restrict__ partial) {
    extern __shared__ uint32_t lds_max[];
    const int64_t C = sh.groups, GC = sh.chunks * sh.groups;
    const int64_t gc = blockIdx.x % GC;  // g * C + c
    const int64_t b = blockIdx.x / GC;
    const int c = (int)(gc % C);
    const int64_t g = gc / C;
    const int H = (int)sh.heads, D = (int)sh.head_dim;
    const int64_t row_len = sh.heads * sh.head_dim;
    constexpr int VEC = IO::VEC;
    const int npos = (int)(row_len / VEC);
    const int64_t r0 = g * sh.rpc;
    const int64_t r1 = r0 + sh.rpc < sh.seq ? r0 + sh.rpc : sh.seq;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int h = threadIdx.x; h < H; h += 256) lds_max[h] = 0u;
    __syncthreads();
    // Lanes past the row re-read its last position: a duplicate does not
    // change a maximum, and unpredicated loads stay in flight together.
    int off[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const int pos = c * 64 * NS + lane + 64 * i;
        off[i] = (pos < npos ? pos : npos - 1) * VEC;
    }
    uint32_t m[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) m[i] = 0u;
    const uint16_t* xb = x + b * sh.seq * row_len;
    for (int64_t row = r0 + wave; row < r1; row += 4) {
        const uint16_t* xr = xb + row * row_len;
        typename IO::T v[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i) v[i] = IO::load(xr + off[i]);
#pragma unroll
        for (int i = 0; i < NS; ++i) m[i] = IO::amax_bits(m[i], v[i]);
    }
#pragma unroll
    for (int i = 0; i < NS; ++i)
        if (c * 64 * NS + lane + 64 * i < npos) atomicMax(&lds_max[off[i] / D], __float_as_uint(amax_from_packed(m[i])));
    __syncthreads();
    for (int h = threadIdx.x; h < H; h += 256) partial[(b * sh.heads + h) * GC + gc] = __uint_as_float(lds_max[h]);
}

// Pass 2.  One wavefront per (b, h) = blockIdx.x * 4 + wave; n = G * C <= 1024
// partials each.  Lanes past n re-read the last one (loads stay unpredicated
// and in flight together).
__global__ __launch_bounds__(256) void head_scale_kernel(const float* __restrict__ partial, int64_t pairs, int n,
                                                         float* __restrict__ scale_out) {
    const int64_t bh = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (bh >= pairs) return;
    const int lane = threadIdx.x & 63;
    const float* p = partial + bh * n;
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int i = lane + 64 * k;
        v[k] = p[i < n ? i : n - 1];
    }
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) a = mag_max(a, v[k]);
    a = wave_max(a);
    if (lane == 0) scale_out[bh] = amax_scale(a, kE4M3Recip);
}

// Pass 3.  blockIdx.x = (b * G + g) * C + c.
template <class IO, int NS>
__global__ __launch_bounds__(256) void head_quant_kernel(const uint16_t* __restrict__ x, HeadQuantShape sh,
                                                         const float* __restrict__ scales,
                                                         uint8_t* __restrict__ q) {
    const int64_t C = sh.groups, GC = sh.chunks * sh.groups;
    const int64_t gc = blockIdx.x % GC;
    const int64_t b = blockIdx.x / GC;
    const int c = (int)(gc % C);
    const int64_t g = gc / C;
    const int D = (int)sh.head_dim;
    const int64_t row_len = sh.heads * sh.head_dim;
    constexpr int VEC = IO::VEC;
    const int npos = (int)(row_len / VEC);
    const int64_t r0 = g * sh.rpc;
    const int64_t r1 = r0 + sh.rpc < sh.seq ? r0 + sh.rpc : sh.seq;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint16_t* xb = x + b * sh.seq * row_len;
    uint8_t* qb = q + b * sh.seq * row_len;
    const float* sb = scales + b * sh.heads;
    int off[NS];
    HeadQuant rq[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const int pos = c * 64 * NS + lane + 64 * i;
        off[i] = (pos < npos ? pos : npos - 1) * VEC;
        rq[i].set(sb[off[i] / D]);
    }
    for (int64_t row = r0 + wave; row < r1; row += 4) {
        const uint16_t* xr = xb + row * row_len;
        uint8_t* qr = qb + row * row_len;
        typename IO::T v[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i) v[i] = IO::load(xr + off[i]);
#pragma unroll
        for (int i = 0; i < NS; ++i)
            if (c * 64 * NS + lane + 64 * i < npos) IO::store(qr + off[i], v[i], rq[i]);
    }
}

namespace {

constexpr int kMaxSlots = 8;  // positions per lane of a column group

// Positions of a row: 16-byte vectors when head_dim % 8 == 0, else elements.
int64_t row_positions(int64_t heads, int64_t head_dim) {
    return heads * head_dim / (head_dim % 8 == 0 ? 8 : 1);
}

HeadQuantShape head_quant_shape(int64_t batch, int64_t seq, int64_t heads, int64_t head_dim) {
    HeadQuantShape sh{};
    sh.batch = batch;
    sh.seq = seq;
    sh.heads = heads;
    sh.head_dim = head_dim;
    const int64_t per_lane = (row_positions(heads, head_dim) + 63) / 64;
    sh.groups = (per_lane + kMaxSlots - 1) / kMaxSlots;
    // About 2048 workgroups of four row-wavefronts in passes 1 and 3, at
    // least 16 rows per workgroup, G * C <= 1024 partials per head.
    int64_t g = (2048 + batch * sh.groups - 1) / (batch * sh.groups);
    const int64_t by_rows = (seq + 15) / 16;
    if (g > by_rows) g = by_rows;
    if (g * sh.groups > 1024) g = 1024 / sh.groups;
    if (g < 1) g = 1;
    sh.rpc = (seq + g - 1) / g;
    sh.chunks = (seq + sh.rpc - 1) / sh.rpc;
    return sh;
}

template <class IO, int NS>
hipError_t launch_head_quant_ns(const uint16_t* x, const HeadQuantShape& sh, float* partial, uint8_t* q,
                                float* scales, hipStream_t st) {
    const dim3 grid((unsigned)(sh.batch * sh.chunks * sh.groups)), blk(256);
    hipLaunchKernelGGL((head_amax_kernel<IO, NS>), grid, blk, (size_t)sh.heads * 4, st, x, sh, partial);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t pairs = sh.batch * sh.heads;
    hipLaunchKernelGGL(head_scale_kernel, dim3((unsigned)((pairs + 3) / 4)), blk, 0, st, (const float*)partial,
                       pairs, (int)(sh.chunks * sh.groups), scales);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((head_quant_kernel<IO, NS>), grid, blk, 0, st, x, sh, (const float*)scales, q);
    return hipGetLastError();
}

template <class IO>
hipError_t launch_head_quant(const uint16_t* x, const HeadQuantShape& sh, float* partial, uint8_t* q,
                             float* scales, hipStream_t st) {
    // Positions per lane of a column group: the row's positions spread evenly
    // over the C groups.
    const int64_t per_lane = (row_positions(sh.heads, sh.head_dim) + 63) / 64;
    const int64_t ns = (per_lane + sh.groups - 1) / sh.groups;
    switch (ns) {
        case 1: return launch_head_quant_ns<IO, 1>(x, sh, partial, q, scales, st);
        case 2: return launch_head_quant_ns<IO, 2>(x, sh, partial, q, scales, st);
        case 3: return launch_head_quant_ns<IO, 3>(x, sh, partial, q, scales, st);
        case 4: return launch_head_quant_ns<IO, 4>(x, sh, partial, q, scales, st);
        case 5: return launch_head_quant_ns<IO, 5>(x, sh, partial, q, scales, st);
        case 6: return launch_head_quant_ns<IO, 6>(x, sh, partial, q, scales, st);
        case 7: return launch_head_quant_ns<IO, 7>(x, sh, partial, q, scales, st);
        default: return launch_head_quant_ns<IO, kMaxSlots>(x, sh, partial, q, scales, st);
    }
}

}  // namespace

int64_t per_head_quant_parts(int64_t batch, int64_t seq, int64_t heads, int64_t head_dim) {
    const HeadQuantShape sh = head_quant_shape(batch, seq, heads, head_dim);
    return batch * heads * sh.chunks * sh.groups;
}

hipError_t launch_quant_per_head_e4m3(const uint16_t* x, int64_t batch, int64_t seq, int64_t heads,
                                      int64_t head_dim, float* partial, uint8_t* q, float* scales,
                                      hipStream_t st) {
    // The shape (and the workspace size) depends on head_dim % 8 only; a
    // misaligned x or q keeps the 8-element positions with scalar accesses.
    const HeadQuantShape sh = head_quant_shape(batch, seq, heads, head_dim);
    if (head_dim % 8) return launch_head_quant<IoElem>(x, sh, partial, q, scales, st);
    if ((uintptr_t)x % 16 == 0 && (uintptr_t)q % 8 == 0) return launch_head_quant<IoVec>(x, sh, partial, q, scales, st);
    return launch_head_quant<IoVecUnaligned>(x, sh, partial, q, scales, st);
}

}  // namespace h3q
