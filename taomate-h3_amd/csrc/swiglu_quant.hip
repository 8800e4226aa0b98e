// Fused SwiGLU + per-token quantization, gfx950: the producer of the fc2 input
// of a DiT MLP (H3/model/layers.py:469-479: F.silu(gate) * up, or the Triton
// fused_swiglu of H3/inference/fused_kernels.py:240-261, 663-677), with the
// activation quantizer of the following W8A8 linear folded in.  For a row
// [gate (F) | up (F)] of bf16:
//
//   e = exp(-gate)
//   s = bf16(gate / (1 + e))           (IEEE binary32 sum and division: torch's
//                                       silu, x / (1 + exp(-x)), rounded to bf16)
//   y = bf16(s * up)                   (stored if out)
//   codes, s_row = per-token quantization of y   (if codes)
//
// s depends on gate alone, through 65536 possible bf16 values.  The
// definition of e is exp_f32 of the CPU restatement (Cody and Waite reduction
// and a degree-7 polynomial from IEEE operations only, within 1 ulp of a
// correctly rounded exp); the kernel evaluates e with the hardware exp2
// (v_exp_f32 of -gate * RN(1/ln 2)), and s comes out bit-identical to the
// restatement's for every one of the 65536 bf16 gate values (checked
// exhaustively on MI355X, tests/test_gpu_swiglu.py), at 2 instructions instead
// of about 15 and two branches.  The sum, the division and the products are
// single IEEE operations in the order written, so the CPU restatement
// reproduces y bit for bit.  The reference's results differ from these only
// where its own exp (the library's, or Triton's) moves the binary32 silu
// across a bf16 rounding boundary.
//
// One wavefront per row, y kept in VGPRs (NV 8-element vectors per lane) for
// the quantizer; gate and up are read in batches of four vectors per lane.
// Per row 4F bytes in, F bytes of codes + 4 bytes of scale out (+ 2F with out).
//
// Table form (swiglu_quant_lut_kernel, calls of at least kLutMinRows rows).
// Because s is a function of the 16-bit gate pattern alone, the library
// evaluates it once per device for all 65536 patterns (silu_table_kernel,
// the same instructions as above) into a 128 KiB table in device memory.
// Each workgroup copies the table into LDS when it starts and looks s up
// there (one LDS read per element instead of the exp, the sum and the IEEE
// division), so the outputs are the same bits and the kernel sheds about
// half of its vector instructions.  The first call on a device fills the
// table and waits for it (once); a call made while its stream is being
// captured into a graph before that has happened runs the form above.
#include <mutex>

#include "h3q_common.hpp"
#include "h3q_kernels.hpp"
#include "row_quant.hpp"

#pragma clang fp contract(off)

namespace h3q {

namespace {

__device__ __forceinline__ float silu_f32(float g) {
    const float e = __builtin_amdgcn_exp2f(-g * 0x1.715476p+0f);  // exp(-g)
    return g / (1.0f + e);
}

// Two gate and two up values (packed bf16) -> two y values (packed bf16).
__device__ __forceinline__ uint32_t swiglu2(uint32_t g, uint32_t u) {
    const uint32_t s = pack_bf16x2(silu_f32(bf16_lo(g)), silu_f32(bf16_hi(g)));
    return pack_bf16x2(bf16_lo(s) * bf16_lo(u), bf16_hi(s) * bf16_hi(u));
}

// The same with s read from the LDS table (indexed by the gate's bits).
__device__ __forceinline__ uint32_t swiglu2_lut(const H3Q_LDS uint16_t* t, uint32_t g, uint32_t u) {
    const uint32_t s = (uint32_t)t[g & 0xFFFFu] | ((uint32_t)t[g >> 16] << 16);
    return pack_bf16x2(bf16_lo(s) * bf16_lo(u), bf16_hi(s) * bf16_hi(u));
}

}  // namespace

// bf16(silu(g)) for every 16-bit pattern g, one per device (see above).
__device__ __align__(256) uint16_t silu_table[65536];

__global__ __launch_bounds__(256) void silu_table_kernel(uint16_t* __restrict__ table) {
    const uint32_t g = (blockIdx.x * 256 + threadIdx.x) * 2;
    // the pair (g, g + 1) as one packed word, rounded exactly as swiglu2 does
    const uint32_t w = g | ((g + 1) << 16);
    reinterpret_cast<uint32_t*>(table)[g >> 1] = pack_bf16x2(silu_f32(bf16_lo(w)), silu_f32(bf16_hi(w)));
}

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

// Table form: one workgroup of LUT_WAVES waves per CU (the 128 KiB table
// fills most of the LDS), rows dealt to waves in order as above.
constexpr int kLutWaves = 8;
template <int FMT, int ROUND, int NV>
__global__ __launch_bounds__(kLutWaves * 64) void swiglu_quant_lut_kernel(SwigluQuantArgs p,
                                                                         const uint16_t* __restrict__ table) {
    __shared__ __attribute__((aligned(1024))) uint16_t lds_table[65536];
    {
        // 128 KiB by LDS-DMA: 128 wave copies of 1 KiB, 16 per wave.
        const CopySrc src(table, 65536u * 2u);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
        const uint32_t base = (uint32_t)(uintptr_t)(H3Q_LDS uint16_t*)lds_table;
#pragma unroll
        for (int i = 0; i < 128 / kLutWaves; ++i) {
            const int c = wave + kLutWaves * i;
            copy16(src, base + (uint32_t)(c * 1024), (uint32_t)(c * 1024 + 16 * lane));
        }
        wait_vmcnt0();
        __syncthreads();
    }
    const H3Q_LDS uint16_t* t = (const H3Q_LDS uint16_t*)lds_table;
    const int lane = threadIdx.x & 63;
    const int nvec = p.half >> 3;
    const int64_t step = (int64_t)gridDim.x * kLutWaves;
    for (int64_t row = (int64_t)blockIdx.x * kLutWaves + (threadIdx.x >> 6); row < p.rows; row += step) {
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
                y[i0 + b] = make_uint4(swiglu2_lut(t, g[b].x, u[b].x), swiglu2_lut(t, g[b].y, u[b].y),
                                       swiglu2_lut(t, g[b].z, u[b].z), swiglu2_lut(t, g[b].w, u[b].w));
                // as above: keeps the compiler from holding many vectors' lookups live at once
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

// Calls of at least this many rows take the table form (below it the
// table's copy into every workgroup's LDS is not paid back).
constexpr int64_t kLutMinRows = 1024;

// The current device's table, filled on first use (launch + wait, once per
// device), and its CU count; null while a graph is being captured on st and
// the table does not exist yet.
hipError_t silu_table_for(hipStream_t st, const uint16_t** out, int* cus) {
    constexpr int kMaxDevices = 64;
    static std::mutex lock;
    static const uint16_t* tables[kMaxDevices] = {};
    static int cu_count[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(lock);
    if (!tables[dev]) {
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &status);
        if (e != hipSuccess) return e;
        if (status != hipStreamCaptureStatusNone) {
            *out = nullptr;
            return hipSuccess;
        }
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(silu_table));  // the current device's copy
        if (e != hipSuccess) return e;
        e = hipDeviceGetAttribute(&cu_count[dev], hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        // The wait below is legal even while another stream of this thread
        // is being captured in global mode: relaxed mode for the fill only.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(silu_table_kernel, dim3(65536 / 512), dim3(256), 0, st, (uint16_t*)ptr);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        const hipError_t restore = hipThreadExchangeStreamCaptureMode(&mode);
        if (e == hipSuccess) e = restore;
        if (e != hipSuccess) return e;
        tables[dev] = (const uint16_t*)ptr;
    }
    *out = tables[dev];
    *cus = cu_count[dev] > 0 ? cu_count[dev] : 256;
    return hipSuccess;
}

template <int FMT, int ROUND, int NV>
hipError_t launch_sq_nv(const SwigluQuantArgs& a, hipStream_t st) {
    // (the widest rows, NV = 32, would spill registers in the table form)
    if constexpr (NV <= 28) {
        if (a.rows >= kLutMinRows) {
            const uint16_t* table = nullptr;
            int cus = 0;
            const hipError_t e = silu_table_for(st, &table, &cus);
            if (e != hipSuccess) return e;
            if (table) {
                const int64_t waves = (a.rows + kLutWaves - 1) / kLutWaves;
                const int64_t blocks = waves < cus ? waves : cus;
                hipLaunchKernelGGL((swiglu_quant_lut_kernel<FMT, ROUND, NV>), dim3((unsigned)blocks),
                                   dim3(kLutWaves * 64), 0, st, a, table);
                return hipGetLastError();
            }
        }
    }
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
    if (nvec <= 1728) return launch_sq_nv<FMT, ROUND, 27>(a, st);  // F = 13824 exactly
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
