// Weight-streaming scaled GEMM for few activation rows (M <= 128) on gfx950.
//
//   out[m, n] = bf16( s_a[m] * (s_w[n] * sum_k A[m, k] * W[n, k]) [+ bias[n]] )
//
// With M this small the GEMM is bound by reading W [N, K] once from HBM
// (N * K bytes), not by the MFMAs.  So the weight goes straight from HBM into
// MFMA operand registers, without LDS staging, and each workgroup keeps many
// 128-byte weight lines in flight.
//
// Work split.  A workgroup owns 16 * NB weight rows (output columns) and all
// M activation rows (MT tiles of 16).  Its WAVES wavefronts split K: wave w
// takes the 128-byte k-steps w, w + WAVES, ...  Per step a wave needs, for
// each 16-row block of W and of A, a 2 KiB operand tile of
// v_mfma_f32_16x16x128_f8f6f4: row = lane % 16, k = 32 (lane / 16) .. +31.
// That is every row's full 128-byte line for the step.
//
// Pipeline.  Each wave owns a private ring of D LDS slots in this workgroup's
// LDS and fills them with buffer_load_dwordx4 ... lds (HBM -> LDS, no VGPR
// staging).  Copy h (0, 1) of a 16-row block fetches the 16-byte half h of
// every lane's fragment, so the fragment is read back as two conflict-free
// ds_read_b128 at 16 * lane and 1024 + 16 * lane.  The copies are inline asm
// that the compiler does not track, and the wave waits for them with
// explicit vmcnt counts: D - 1 steps stay in flight while one is consumed.
// The ring is private and the slot index is a runtime value, so the loop
// needs no barrier and no register ring.  Steps past K and rows past M or N
// get out-of-range buffer offsets (zeros).  At the end the waves' partial
// accumulators are summed through LDS and the waves share the epilogue.
//
// The weight fragment is the MFMA's A operand, so accumulator slot v of lane
// L holds out[m = 16 t + L % 16][n = n0 + 16 j + 4 (L / 16) + v]: four
// consecutive columns of one row, which are stored as 8 bytes.
//
// int8 uses v_mfma_i32_16x16x64_i8 twice per 32-byte fragment (the low and
// high 16 bytes).  Each k byte meets its partner exactly once, so the sum is
// the full dot product.
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"

namespace h3q {

namespace {

template <int OP>
struct SkinnyMfma;

template <>
struct SkinnyMfma<kOpE4M3> {
    using acc_t = v4f;
    static __device__ __forceinline__ acc_t run(v8i a, v8i b, acc_t c) {
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

template <>
struct SkinnyMfma<kOpInt8> {
    using acc_t = v4i;
    static __device__ __forceinline__ acc_t run(v8i a, v8i b, acc_t c) {
        const v4i alo = {a[0], a[1], a[2], a[3]}, ahi = {a[4], a[5], a[6], a[7]};
        const v4i blo = {b[0], b[1], b[2], b[3]}, bhi = {b[4], b[5], b[6], b[7]};
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, blo, c, 0, 0, 0);
        return __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, bhi, c, 0, 0, 0);
    }
};

constexpr uint32_t kOob = 0x80000000u;  // beyond every descriptor's range: loads return 0, stores drop
// Cache policy of the tiled weight loads: non-temporal.  Every weight byte is
// read once per call, so keeping it in the L2 only evicts the activations,
// which every workgroup re-reads.  Measured at c4 (two alternating runs):
// M = 16 7.67 -> 7.26 us, M = 64 11.3 -> 10.8 us, M = 128 15.0 -> 14.7 us.
constexpr int kWeightLoadPolicy = 2;

}  // namespace

// Shared epilogue: red holds each wave's partial accumulators, indexed
// ((wave * NB + j) * MT + t) * 64 + lane; wave w finishes the (j, t) tiles with
// (j * MT + t) % WAVES == w: the sum over waves, then s_a * (s_w * acc) [+ bias]
// to bf16, four consecutive columns per 8-byte store.
// Epilogue vectors, copied into LDS by LDS-DMA when the kernel starts (so
// the epilogue needs no memory round trip after the last MFMA): bytes
// [0, 1024) the column scales of the workgroup's 16 * NB columns (or the
// per-tensor scale), [1024, 1536) their bias, [1536, 2048) the row scales.
// Buffer loads check their range per dword: a dword past the end reads 0.
constexpr int kSkinnyVecBytes = 2048;
template <int NB>
__device__ __forceinline__ void skinny_vectors(const GemmArgs& p, H3Q_LDS uint8_t* vec, int64_t n0, int wave,
                                               int lane, bool with_bias) {
    const int64_t cols = (p.n - n0) < 16 * NB ? (p.n - n0) : 16 * NB;
    const uint32_t base = (uint32_t)(uintptr_t)vec;
    if (wave != 0) return;  // some configurations have only two waves
    copy16(CopySrc(p.b_scale + (p.b_scale_per_col ? n0 : 0), (uint32_t)(p.b_scale_per_col ? cols : 1) * 4u), base,
           16u * lane);
    if (with_bias)
        copy16(CopySrc(p.bias + n0, (uint32_t)cols * 2u), base + 1024u, lane < 32 ? 16u * lane : 0x80000000u);
    copy16(CopySrc(p.a_scale, (uint32_t)(p.a_scale_per_row ? p.m : 1) * 4u), base + 1536u,
           lane < 32 ? 16u * lane : 0x80000000u);
}

template <class acc_t, int MT, int NB, int WAVES, bool VEC, bool BIAS>
__device__ __forceinline__ void skinny_epilogue(const GemmArgs& p, const H3Q_LDS uint8_t* vec,
                                                const H3Q_LDS acc_t* red, int64_t n0, int wave, int lane) {
    const H3Q_LDS float* vsw = (const H3Q_LDS float*)vec;
    const H3Q_LDS uint16_t* vbias = (const H3Q_LDS uint16_t*)(vec + 1024);
    const H3Q_LDS float* vsa = (const H3Q_LDS float*)(vec + 1536);
    const int r16 = lane & 15, kq = lane >> 4;
    const int64_t ldo = p.ldo;
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.out, (uint32_t)(p.m * ldo * 2));
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int64_t n = n0 + 16 * j + 4 * kq;  // first of this lane's four columns
        float sw[4], bias[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool in = n + e < p.n;
            const int nl = (int)(n + e - n0);
            sw[e] = in ? vsw[p.b_scale_per_col ? nl : 0] : 0.0f;
            // The LDS copy drops a dword that straddles the end of the bias
            // (odd column counts, which only the scalar-store variant sees):
            // that variant reads its bias from memory.
            bias[e] = (BIAS || !VEC) && in && p.bias ? out_lo(VEC ? vbias[nl] : p.bias[n + e], p.out_f16) : 0.0f;
        }
        const bool has_bias = VEC ? BIAS : p.bias != nullptr;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if ((j * MT + t) % WAVES != wave) continue;
            acc_t s = red[(j * MT + t) * 64 + lane];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) s += red[((w * NB + j) * MT + t) * 64 + lane];
            const int64_t m = 16 * t + r16;
            const float sa = m < p.m ? vsa[p.a_scale_per_row ? m : 0] : 0.0f;
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = __fmul_rn(sw[e], (float)s[e]);
                y[e] = has_bias ? __builtin_fmaf(sa, v, bias[e]) : __fmul_rn(sa, v);
            }
            const uint32_t w0 = pack_out2(y[0], y[1], p.out_f16), w1 = pack_out2(y[2], y[3], p.out_f16);
            const uint32_t row_off = m < p.m ? (uint32_t)(m * ldo * 2) : kOob;
            if constexpr (VEC) {
                const uint32_t off = (row_off != kOob && n < p.n) ? row_off + (uint32_t)(n * 2) : kOob;
                __builtin_amdgcn_raw_buffer_store_b64(v2u{w0, w1}, ro, off, 0, 0);
            } else {
                const uint16_t h[4] = {(uint16_t)w0, (uint16_t)(w0 >> 16), (uint16_t)w1, (uint16_t)(w1 >> 16)};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t off =
                        (row_off != kOob && n + e < p.n) ? row_off + (uint32_t)((n + e) * 2) : kOob;
                    __builtin_amdgcn_raw_buffer_store_b16(h[e], ro, off, 0, 0);
                }
            }
        }
    }
}

template <int OP, int MT, int NB, int WAVES, int D, bool VEC, bool BIAS>
__global__ __launch_bounds__(WAVES * 64) void skinny_kernel(GemmArgs p) {
    using acc_t = typename SkinnyMfma<OP>::acc_t;
    constexpr int BN = 16 * NB;
    constexpr int PARTS = NB + MT;          // 2 KiB operand tiles per step
    constexpr int SLOT = PARTS * 2048;
    constexpr int LPS = 2 * PARTS;          // copy instructions per step
    static_assert((D - 1) * LPS < 64, "vmcnt range");
    constexpr int RING = WAVES * D * SLOT;
    constexpr int RED = WAVES * NB * MT * 64 * (int)sizeof(acc_t);
    __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[RING > RED ? RING : RED];
    __shared__ __attribute__((aligned(16))) uint8_t lds_vec[kSkinnyVecBytes];
    H3Q_LDS uint8_t* const lds = (H3Q_LDS uint8_t*)lds_raw;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, kq = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * BN;
    const int64_t kbytes = p.k;
    const int64_t rows_b = (p.n - n0) < BN ? (p.n - n0) : BN;
    const CopySrc rw((const uint8_t*)p.b + n0 * p.ldb, (uint32_t)(rows_b * p.ldb));
    const CopySrc rx(p.a, (uint32_t)(p.m * p.lda));

    skinny_vectors<NB>((const GemmArgs&)p, (H3Q_LDS uint8_t*)lds_vec, n0, wave, lane, (BIAS || !VEC) && p.bias);
    uint32_t woff[NB], xoff[MT];
#pragma unroll
    for (int j = 0; j < NB; ++j) woff[j] = 16 * j + r16 < rows_b ? (uint32_t)((16 * j + r16) * p.ldb) : kOob;
#pragma unroll
    for (int t = 0; t < MT; ++t) xoff[t] = 16 * t + r16 < p.m ? (uint32_t)((16 * t + r16) * p.lda) : kOob;

    H3Q_LDS uint8_t* const ring = lds + wave * D * SLOT;
    const int steps = (int)((kbytes + 127) / 128);
    const int iters = (steps + WAVES - 1) / WAVES;
    // Copy step i of this wave (k bytes [128 (i WAVES + wave), +128)) into slot.
    auto issue = [&](int i, int slot) {
        const int64_t k = (int64_t)(i * WAVES + wave) * 128 + 32 * kq;
        const uint32_t base = (uint32_t)(uintptr_t)(ring + slot * SLOT);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool in = k + 16 * h < kbytes;
#pragma unroll
            for (int j = 0; j < NB; ++j)
                copy16(rw, base + (2 * j + h) * 1024, in ? woff[j] + (uint32_t)(k + 16 * h) : kOob);
#pragma unroll
            for (int t = 0; t < MT; ++t)
                copy16(rx, base + (2 * (NB + t) + h) * 1024, in ? xoff[t] + (uint32_t)(k + 16 * h) : kOob);
        }
    };
    auto frag = [&](const H3Q_LDS uint8_t* tile) -> v8i {
        const v4i lo = *(const H3Q_LDS v4i*)(tile + 16 * lane);
        const v4i hi = *(const H3Q_LDS v4i*)(tile + 1024 + 16 * lane);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    acc_t acc[NB][MT];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = acc_t{};

#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
    int slot = 0;
    for (int i = 0; i < iters; ++i) {
        wait_vmcnt<(D - 1) * LPS>();
        asm volatile("" ::: "memory");
        const H3Q_LDS uint8_t* cur = ring + slot * SLOT;
        v8i wf[NB], xf[MT];
#pragma unroll
        for (int j = 0; j < NB; ++j) wf[j] = frag(cur + 2 * j * 1024);
#pragma unroll
        for (int t = 0; t < MT; ++t) xf[t] = frag(cur + 2 * (NB + t) * 1024);
        // The slot's reads must have completed before its refill is issued.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(i + D, slot);
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[j][t] = SkinnyMfma<OP>::run(wf[j], xf[t], acc[j][t]);
        slot = slot + 1 == D ? 0 : slot + 1;
    }
    wait_vmcnt<0>();
    __syncthreads();  // every wave is done with the ring before it is reused below

    // Sum the waves' partial accumulators through LDS (reusing the ring); wave
    // w then finishes the (j, t) tiles with (j * MT + t) % WAVES == w.
    H3Q_LDS acc_t* const red = (H3Q_LDS acc_t*)lds;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) red[((wave * NB + j) * MT + t) * 64 + lane] = acc[j][t];
    __syncthreads();

    skinny_epilogue<acc_t, MT, NB, WAVES, VEC, BIAS>(p, (const H3Q_LDS uint8_t*)lds_vec, red, n0, wave, lane);
}

// Skinny GEMM over a tiled weight (and optionally tiled activations).  In the
// tiled layout the 16-row x 128-byte operand tile of one MFMA step is 2 KiB
// contiguous in fragment order, so each half of a fragment is one fully
// coalesced 1 KiB load straight into VGPRs.  A workgroup owns 16 * NB weight
// rows; its waves split K (wave w takes steps w, w + WAVES, ...).  Each wave
// works in chunks of SPW steps: it issues a chunk's loads (W and A) before
// the chunk's first MFMA (sched_barrier keeps the compiler from sinking them
// next to their uses), so a chunk costs one memory round trip; with PIPE two
// register sets hold chunks c and c + 1, and chunk c + 1's loads are issued
// before chunk c's MFMAs, so the round trips overlap.  Row-major
// activations use the fragment mapping directly (row = lane % 16, 32 bytes at
// 32 (lane / 16)).
template <int OP, int MT, int NB, int WAVES, int SPW, bool PIPE, bool A_TILED, bool VEC, bool BIAS>
__global__ __launch_bounds__(WAVES * 64) void skinny_tiled_kernel(GemmArgs p) {
    using acc_t = typename SkinnyMfma<OP>::acc_t;
    __shared__ __attribute__((aligned(16))) acc_t red[WAVES * NB * MT * 64];
    __shared__ __attribute__((aligned(16))) uint8_t lds_vec[kSkinnyVecBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, kq = lane >> 4;
    const int64_t blk0 = (int64_t)blockIdx.x * NB;        // first 16-row weight block
    const int64_t n0 = blk0 * 16;
    const int64_t kbytes = p.k, steps = kbytes / 128;
    const int64_t blocks_b = (p.n + 15) / 16;
    const int64_t nblk = (blocks_b - blk0) < NB ? (blocks_b - blk0) : NB;
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc((const uint8_t*)p.b + blk0 * steps * 2048, (uint32_t)(nblk * steps * 2048));
    const int64_t a_bytes = A_TILED ? (p.m + 15) / 16 * steps * 2048 : p.m * p.lda;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.a, (uint32_t)a_bytes);

    skinny_vectors<NB>(p, (H3Q_LDS uint8_t*)lds_vec, n0, wave, lane, (BIAS || !VEC) && p.bias);
    uint32_t xoff[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        if constexpr (A_TILED) xoff[t] = 16 * t < p.m ? (uint32_t)(t * steps * 2048 + 16 * lane) : kOob;
        else xoff[t] = 16 * t + r16 < p.m ? (uint32_t)((16 * t + r16) * p.lda + 32 * kq) : kOob;
    }
    const int iters = (int)((steps + WAVES - 1) / WAVES);

    acc_t acc[NB][MT];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = acc_t{};

    // Chunk c: this wave's steps c * SPW .. c * SPW + SPW - 1 (step st at k
    // bytes 128 st, st = chunk step * WAVES + wave); steps past K load zeros.
    auto load_chunk = [&](int c, v8i (&wf)[SPW][NB], v8i (&xf)[SPW][MT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int64_t st = (int64_t)(c * SPW + i) * WAVES + wave;
            const bool in = st < steps;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const uint32_t o = in && j < nblk ? (uint32_t)((j * steps + st) * 2048 + 16 * lane) : kOob;
                const v4u lo =
                    __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, kWeightLoadPolicy));
                const v4u hi = __builtin_bit_cast(
                    v4u, __builtin_amdgcn_raw_buffer_load_b128(rw, o == kOob ? kOob : o + 1024, 0, kWeightLoadPolicy));
                wf[i][j] = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                uint32_t o0 = kOob, o1 = kOob;
                if (in && xoff[t] != kOob) {
                    if constexpr (A_TILED) {
                        o0 = xoff[t] + (uint32_t)(st * 2048);
                        o1 = o0 + 1024;
                    } else {
                        o0 = xoff[t] + (uint32_t)(st * 128);
                        o1 = o0 + 16;
                    }
                }
                const v4u lo = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, o0, 0, 0));
                const v4u hi = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, o1, 0, 0));
                xf[i][t] = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            }
        }
    };
    auto mfma_chunk = [&](const v8i (&wf)[SPW][NB], const v8i (&xf)[SPW][MT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < SPW; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[j][t] = SkinnyMfma<OP>::run(wf[i][j], xf[i][t], acc[j][t]);
    };
    const int nc = (iters + SPW - 1) / SPW;
    if constexpr (PIPE) {
        // Two register sets: the next chunk's loads are issued before the
        // current chunk's MFMAs (sched_barrier keeps them there, and the
        // compiler's vmcnt waits then leave the newer chunk in flight).  The
        // last one or two chunks are peeled, so no load is issued past the
        // end and every wait sits in straight-line code.
        v8i wa[SPW][NB], xa[SPW][MT], wb[SPW][NB], xb[SPW][MT];
        load_chunk(0, wa, xa);
        int c = 0;
        for (; c + 2 < nc; c += 2) {
            load_chunk(c + 1, wb, xb);
            __builtin_amdgcn_sched_barrier(0);
            mfma_chunk(wa, xa);
            load_chunk(c + 2, wa, xa);
            __builtin_amdgcn_sched_barrier(0);
            mfma_chunk(wb, xb);
        }
        if (c + 1 < nc) {
            load_chunk(c + 1, wb, xb);
            __builtin_amdgcn_sched_barrier(0);
            mfma_chunk(wa, xa);
            mfma_chunk(wb, xb);
        } else {
            mfma_chunk(wa, xa);
        }
    } else {
        // One register set: each chunk's loads, then its MFMAs (one round
        // trip per chunk; with SPW * WAVES >= K / 128 there is one chunk).
        for (int c = 0; c < nc; ++c) {
            v8i wf[SPW][NB], xf[SPW][MT];
            load_chunk(c, wf, xf);
            __builtin_amdgcn_sched_barrier(0);
            mfma_chunk(wf, xf);
        }
    }

#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) red[((wave * NB + j) * MT + t) * 64 + lane] = acc[j][t];
    wait_vmcnt0();  // the epilogue vectors' LDS copies (not tracked by the compiler)
    __syncthreads();
    skinny_epilogue<acc_t, MT, NB, WAVES, VEC, BIAS>(p, (const H3Q_LDS uint8_t*)lds_vec, (const H3Q_LDS acc_t*)red,
                                                     n0, wave, lane);
}

namespace {

template <int OP, int MT, int NB, int WAVES, int D>
hipError_t launch_skinny_cfg(const GemmArgs& a, hipStream_t st) {
    const unsigned blocks = (unsigned)((a.n + 16 * NB - 1) / (16 * NB));
    if (!a.out_vec)
        hipLaunchKernelGGL((skinny_kernel<OP, MT, NB, WAVES, D, false, false>), dim3(blocks), dim3(WAVES * 64), 0,
                           st, a);
    else if (a.bias)
        hipLaunchKernelGGL((skinny_kernel<OP, MT, NB, WAVES, D, true, true>), dim3(blocks), dim3(WAVES * 64), 0, st,
                           a);
    else
        hipLaunchKernelGGL((skinny_kernel<OP, MT, NB, WAVES, D, true, false>), dim3(blocks), dim3(WAVES * 64), 0,
                           st, a);
    return hipGetLastError();
}

template <int OP, int MT, int NB, int WAVES, int SPW, bool PIPE, bool A_TILED>
hipError_t launch_tiled_cfg(const GemmArgs& a, hipStream_t st) {
    const unsigned blocks = (unsigned)(((a.n + 15) / 16 + NB - 1) / NB);
    if (!a.out_vec)
        hipLaunchKernelGGL((skinny_tiled_kernel<OP, MT, NB, WAVES, SPW, PIPE, A_TILED, false, false>), dim3(blocks),
                           dim3(WAVES * 64), 0, st, a);
    else if (a.bias)
        hipLaunchKernelGGL((skinny_tiled_kernel<OP, MT, NB, WAVES, SPW, PIPE, A_TILED, true, true>), dim3(blocks),
                           dim3(WAVES * 64), 0, st, a);
    else
        hipLaunchKernelGGL((skinny_tiled_kernel<OP, MT, NB, WAVES, SPW, PIPE, A_TILED, true, false>), dim3(blocks),
                           dim3(WAVES * 64), 0, st, a);
    return hipGetLastError();
}

// Configurations measured on MI355X at N = K = 5120 (tiled weight and
// activations, 12 rotating weight copies): 32 weight rows per workgroup beat
// 16 once M >= 64 (each workgroup re-reads all of A from L2, so fewer
// workgroups move fewer bytes): M = 64 11.6 us vs 15.0 us, M = 128 16.0 us vs
// 20.5 us.  Pipelined chunks: M = 64 11.3 us, M = 128 15.1 us with single-step
// chunks (against 11.6 and 15.8 without); M = 16 7.7 us with two chunks of 5
// steps (against 7.9 us in one chunk of 10).  Non-temporal weight loads then
// took M = 16 / 64 / 128 to 7.26 / 10.8 / 14.7 us.
template <int OP, bool A_TILED>
hipError_t launch_tiled_op(const GemmArgs& a, hipStream_t st) {
    if (a.m <= 16) return launch_tiled_cfg<OP, 1, 2, 4, 5, true, A_TILED>(a, st);
    if (a.m <= 32) return launch_tiled_cfg<OP, 2, 2, 8, 5, false, A_TILED>(a, st);
    if (a.m <= 64) return launch_tiled_cfg<OP, 4, 2, 8, 1, true, A_TILED>(a, st);
    return launch_tiled_cfg<OP, 8, 2, 8, 1, true, A_TILED>(a, st);
}

// Row-major weights: the LDS-ring kernel above.
template <int OP>
hipError_t launch_skinny_op(const GemmArgs& a, hipStream_t st) {
    if (a.b_tiled) return a.a_tiled ? launch_tiled_op<OP, true>(a, st) : launch_tiled_op<OP, false>(a, st);
    if (a.m <= 16) return launch_skinny_cfg<OP, 1, 1, 4, 5>(a, st);
    if (a.m <= 32) return launch_skinny_cfg<OP, 2, 1, 4, 3>(a, st);
    if (a.m <= 64) return launch_skinny_cfg<OP, 4, 1, 2, 4>(a, st);
    return launch_skinny_cfg<OP, 8, 1, 2, 2>(a, st);
}

}  // namespace

bool skinny_supported(const GemmArgs& a) {
    const int64_t a_bytes = a.a_tiled ? (a.m + 15) / 16 * (a.k / 128) * 2048 : a.m * a.lda;
    return a.m >= 1 && a.m <= kSkinnyMaxM && a.lora_t == nullptr && a_bytes < (int64_t)kOob &&
           a.m * a.ldo * 2 < (int64_t)kOob;
}

hipError_t launch_gemm_skinny(int kind, const GemmArgs& a, hipStream_t st) {
    return kind == kOpInt8 ? launch_skinny_op<kOpInt8>(a, st) : launch_skinny_op<kOpE4M3>(a, st);
}

}  // namespace h3q
