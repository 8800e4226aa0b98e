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
// Two launches.  A scale needs every token of its (batch, head), so the
// input is read twice unless it stays in the caches between the launches:
//
//   head_amax_kernel   workgroup (b, segment of heads, chunk of tokens):
//                      one wave per token row reads the segment's contiguous
//                      bytes (hps heads, about 1 KiB), lanes keep packed
//                      maxima of fixed positions, LDS max per head, one
//                      partial per (b, h, chunk).
//   head_quant_kernel  workgroup (b, w): folds the G partials of each head of
//                      batch b into LDS (scale and RN(1/scale)), then
//                      quantizes tokens w, w + W, ... of batch b; each thread
//                      owns fixed positions of a row, so its heads' scales sit
//                      in registers for all of its rows.
//
// Traffic per element: 2 bytes (pass 1) + 2 + 1 bytes (pass 2); algorithmic
// 3 bytes.  The folds read B * H * G floats per workgroup of pass 2, with
// G * H <= 4096.
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"
#include "row_quant.hpp"

namespace h3q {

namespace {

struct HeadQuantShape {
    int64_t batch, seq, heads, head_dim;
    int64_t hps;     // heads per segment of pass 1
    int64_t nseg;    // segments per row
    int64_t chunks;  // G: token chunks per (batch, segment)
    int64_t rpc;     // tokens per chunk
    int64_t waves2;  // W: pass-2 workgroups per batch
};

constexpr int kMaxHeadsPerSegment = 64;

// Position width in elements: 8 (16-byte vectors) or 1 (single bf16).
template <int VEC>
struct Io;

template <>
struct Io<8> {
    static __device__ __forceinline__ uint32_t amax_bits(const uint16_t* p) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        uint32_t m = pk_abs_max(0u, v.x);
        m = pk_abs_max(m, v.y);
        m = pk_abs_max(m, v.z);
        m = pk_abs_max(m, v.w);
        return m;
    }
    template <class Q>
    static __device__ __forceinline__ void quant(const uint16_t* p, uint8_t* q, const Q& rq) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        uint2 o;
        o.x = rq.pack4(v.x, v.y);
        o.y = rq.pack4(v.z, v.w);
        *reinterpret_cast<uint2*>(q) = o;
    }
};

template <>
struct Io<1> {
    static __device__ __forceinline__ uint32_t amax_bits(const uint16_t* p) { return (uint32_t)(*p & 0x7FFFu); }
    template <class Q>
    static __device__ __forceinline__ void quant(const uint16_t* p, uint8_t* q, const Q& rq) {
        *q = (uint8_t)(rq.pack4((uint32_t)*p, 0u) & 0xFFu);
    }
};

}  // namespace

// Pass 1.  blockIdx.x = (b * nseg + seg) * G + g.
template <int VEC, int NS>
__global__ __launch_bounds__(256) void head_amax_kernel(const uint16_t* __restrict__ x, HeadQuantShape sh,
                                                        float* __restrict__ partial) {
    __shared__ uint32_t lds[kMaxHeadsPerSegment];
    const int64_t G = sh.chunks;
    const int64_t g = blockIdx.x % G;
    const int64_t seg = (blockIdx.x / G) % sh.nseg;
    const int64_t b = blockIdx.x / (G * sh.nseg);
    const int64_t h0 = seg * sh.hps;
    const int nh = (int)(sh.heads - h0 < sh.hps ? sh.heads - h0 : sh.hps);
    const int D = (int)sh.head_dim;
    const int sv = nh * D / VEC;  // positions in the segment
    const int64_t row_len = sh.heads * sh.head_dim;
    const int64_t r0 = g * sh.rpc;
    const int64_t r1 = r0 + sh.rpc < sh.seq ? r0 + sh.rpc : sh.seq;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x < (unsigned)nh) lds[threadIdx.x] = 0u;
    __syncthreads();
    const uint16_t* seg_base = x + b * sh.seq * row_len + h0 * sh.head_dim;
    for (int cg = 0; cg < sv; cg += 64 * NS) {
        uint32_t m[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) m[j] = 0u;
#pragma unroll 4
        for (int64_t row = r0 + wave; row < r1; row += 4) {
            const uint16_t* xr = seg_base + row * row_len;
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const int pos = cg + lane + 64 * j;
                if (pos < sv) m[j] = pk_abs_max(m[j], Io<VEC>::amax_bits(xr + pos * VEC));
            }
        }
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const int pos = cg + lane + 64 * j;
            if (pos < sv) atomicMax(&lds[pos * VEC / D], __float_as_uint(amax_from_packed(m[j])));
        }
    }
    __syncthreads();
    if (threadIdx.x < (unsigned)nh) partial[(b * sh.heads + h0 + threadIdx.x) * G + g] = __uint_as_float(lds[threadIdx.x]);
}

// Pass 2.  blockIdx.x = b * W + w.
template <int VEC, int NS>
__global__ __launch_bounds__(256) void head_quant_kernel(const uint16_t* __restrict__ x, HeadQuantShape sh,
                                                         const float* __restrict__ partial,
                                                         uint8_t* __restrict__ q, float* __restrict__ scale_out) {
    // amax[H], then the scales and their reciprocals: 12 * H bytes.
    extern __shared__ uint32_t lds_dyn[];
    uint32_t* amax = lds_dyn;
    float* lds_s = reinterpret_cast<float*>(lds_dyn + sh.heads);
    float* lds_r = lds_s + sh.heads;
    const int64_t W = sh.waves2;
    const int64_t b = blockIdx.x / W;
    const int64_t w = blockIdx.x % W;
    const int H = (int)sh.heads, G = (int)sh.chunks, D = (int)sh.head_dim;
    for (int h = threadIdx.x; h < H; h += 256) amax[h] = 0u;
    __syncthreads();
    const float* pb = partial + b * sh.heads * sh.chunks;
    for (int i = threadIdx.x; i < H * G; i += 256) atomicMax(&amax[i / G], __float_as_uint(pb[i]));
    __syncthreads();
    for (int h = threadIdx.x; h < H; h += 256) {
        const float s = amax_scale(__uint_as_float(amax[h]), kE4M3Recip);
        lds_s[h] = s;
        lds_r[h] = 1.0f / s;
        if (w == 0) scale_out[b * sh.heads + h] = s;
    }
    __syncthreads();

    const int64_t row_len = sh.heads * sh.head_dim;
    const int nvec = (int)(row_len / VEC);
    const uint16_t* xb = x + b * sh.seq * row_len;
    uint8_t* qb = q + b * sh.seq * row_len;
    for (int cg = 0; cg < nvec; cg += 256 * NS) {
        RowQuant<kFmtE4M3, kRoundDiv> rq[NS];
        int pos[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            pos[j] = cg + (int)threadIdx.x + 256 * j;
            const int h = pos[j] < nvec ? pos[j] * VEC / D : 0;
            rq[j].s = lds_s[h];
            rq[j].r = lds_r[h];
        }
#pragma unroll 2
        for (int64_t row = w; row < sh.seq; row += W) {
            const uint16_t* xr = xb + row * row_len;
            uint8_t* qr = qb + row * row_len;
#pragma unroll
            for (int j = 0; j < NS; ++j)
                if (pos[j] < nvec) Io<VEC>::quant(xr + pos[j] * VEC, qr + pos[j] * VEC, rq[j]);
        }
    }
}

namespace {

HeadQuantShape head_quant_shape(int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, bool vec) {
    HeadQuantShape sh{};
    sh.batch = batch;
    sh.seq = seq;
    sh.heads = heads;
    sh.head_dim = head_dim;
    // About 64 positions (1 KiB of bf16 with 16-byte positions) per segment row.
    const int64_t per_seg = (vec ? 512 : 64) / head_dim;
    sh.hps = per_seg < 1 ? 1 : (per_seg > heads ? heads : per_seg);
    if (sh.hps > kMaxHeadsPerSegment) sh.hps = kMaxHeadsPerSegment;
    sh.nseg = (heads + sh.hps - 1) / sh.hps;
    // Chunks: about 1024 workgroups in pass 1, each folded partial set of a
    // batch at most 4096 floats.
    int64_t g = (1024 + batch * sh.nseg - 1) / (batch * sh.nseg);
    const int64_t gmax = 4096 / heads;
    if (g > gmax) g = gmax;
    if (g > 64) g = 64;
    if (g > seq) g = seq;
    if (g < 1) g = 1;
    sh.rpc = (seq + g - 1) / g;
    sh.chunks = (seq + sh.rpc - 1) / sh.rpc;
    int64_t w = (1024 + batch - 1) / batch;
    if (w > seq) w = seq;
    sh.waves2 = w < 1 ? 1 : w;
    return sh;
}

bool head_quant_vec(const void* x, const void* q, int64_t head_dim) {
    return head_dim % 8 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)q % 8 == 0;
}

template <int VEC>
hipError_t launch_head_quant(const uint16_t* x, const HeadQuantShape& sh, float* partial, uint8_t* q,
                             float* scales, hipStream_t st) {
    const int64_t sv = sh.hps * sh.head_dim / VEC;
    const dim3 g1((unsigned)(sh.batch * sh.nseg * sh.chunks)), blk(256);
    if (sv <= 64)
        hipLaunchKernelGGL((head_amax_kernel<VEC, 1>), g1, blk, 0, st, x, sh, partial);
    else if (sv <= 128)
        hipLaunchKernelGGL((head_amax_kernel<VEC, 2>), g1, blk, 0, st, x, sh, partial);
    else
        hipLaunchKernelGGL((head_amax_kernel<VEC, 4>), g1, blk, 0, st, x, sh, partial);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t nvec = sh.heads * sh.head_dim / VEC;
    const dim3 g2((unsigned)(sh.batch * sh.waves2));
    const size_t lds = (size_t)sh.heads * 12;
    if (nvec <= 256)
        hipLaunchKernelGGL((head_quant_kernel<VEC, 1>), g2, blk, lds, st, x, sh, partial, q, scales);
    else if (nvec <= 512)
        hipLaunchKernelGGL((head_quant_kernel<VEC, 2>), g2, blk, lds, st, x, sh, partial, q, scales);
    else if (nvec <= 768)
        hipLaunchKernelGGL((head_quant_kernel<VEC, 3>), g2, blk, lds, st, x, sh, partial, q, scales);
    else
        hipLaunchKernelGGL((head_quant_kernel<VEC, 4>), g2, blk, lds, st, x, sh, partial, q, scales);
    return hipGetLastError();
}

}  // namespace

int64_t per_head_quant_parts(int64_t batch, int64_t seq, int64_t heads, int64_t head_dim) {
    const HeadQuantShape sh = head_quant_shape(batch, seq, heads, head_dim, head_dim % 8 == 0);
    return batch * heads * sh.chunks;
}

hipError_t launch_quant_per_head_e4m3(const uint16_t* x, int64_t batch, int64_t seq, int64_t heads,
                                      int64_t head_dim, float* partial, uint8_t* q, float* scales,
                                      hipStream_t st) {
    const bool vec = head_quant_vec(x, q, head_dim);
    // The workspace size does not depend on alignment: the chunk count only
    // depends on the shape and on head_dim % 8.
    const HeadQuantShape sh = head_quant_shape(batch, seq, heads, head_dim, head_dim % 8 == 0);
    return vec ? launch_head_quant<8>(x, sh, partial, q, scales, st)
               : launch_head_quant<1>(x, sh, partial, q, scales, st);
}

}  // namespace h3q
