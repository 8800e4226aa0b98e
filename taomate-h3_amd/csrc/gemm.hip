// Scaled FP8 / INT8 GEMM (and the bf16 LoRA down-projection) on gfx950 MFMA.
//
//   out[m, n] = epilogue( sum_k A[m, k] * B[n, k] )
//
// A and B are both K-contiguous ("TN": activations [M, K] and nn.Linear
// weights [N, K]).  Block tile BM x BN, four wavefronts in a 2 x 2 grid, each
// owning a (BM/2) x (BN/2) accumulator block of 32 x 32 MFMA tiles:
//   e4m3  v_mfma_f32_32x32x64_f8f6f4   (32 code bytes per lane per operand)
//   int8  v_mfma_i32_32x32x32_i8       (16 bytes per lane)
//   bf16  v_mfma_f32_32x32x16_bf16     (16 bytes per lane)
// K advances in 128-byte tiles.  Each operand tile (rows x 128 B) is copied
// HBM -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging) into one of two
// LDS stages, while the MFMAs consume the other stage.  Inside a stage a row
// is 8 chunks of 16 B stored at chunk ^ (row & 7), so the 8 lanes that share
// a ds_read_b128 phase hit 8 distinct bank groups.  Rows beyond M / N and
// k-chunks beyond K are fetched with an out-of-range buffer offset, which the
// hardware returns as zeros: tails need no special path.
//
// Epilogue (per 32 x 32 tile, in registers):
//   e4m3 / int8: v = s_a[m] * (s_w[n] * float(acc)) [fma(s_a, ., bias[n])]
//                [+ lora_scale * (t[m, :] . lora_b[n, :])  (bf16 MFMA slab)]
//                -> bf16 round-to-nearest-even
//   raw int32:   acc
//   bf16 GEMM:   bf16(acc)
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"

namespace h3q {

constexpr int kBK = 128;  // bytes of K per LDS tile

template <int OP>
struct Mfma;

template <>
struct Mfma<kOpE4M3> {
    using acc_t = v16f;
    using frag_t = v8i;
    static constexpr int kStep = 64;  // k bytes consumed per MFMA
    static __device__ __forceinline__ acc_t run(frag_t a, frag_t b, acc_t c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

template <>
struct Mfma<kOpInt8> {
    using acc_t = v16i;
    using frag_t = v4i;
    static constexpr int kStep = 32;
    static __device__ __forceinline__ acc_t run(frag_t a, frag_t b, acc_t c) {
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<kOpBF16> {
    using acc_t = v16f;
    using frag_t = v4i;
    static constexpr int kStep = 32;
    static __device__ __forceinline__ acc_t run(frag_t a, frag_t b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c,
                                                       0, 0, 0);
    }
};

// Copy rows [0, ROWS) x bytes [k0, k0 + 128) of an operand into an LDS stage.
// One wave instruction fills 1 KiB = 8 rows; lane L lands at byte L * 16 of
// that KiB, i.e. row L / 8, physical chunk L % 8, so it fetches logical chunk
// (L % 8) ^ (L / 8).
template <int ROWS>
__device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t rsrc, H3Q_LDS uint8_t* dst, uint32_t ld,
                                          int64_t k0, int64_t kbytes, int wave, int lane) {
    const int sub = lane >> 3;
    const int lch = (lane & 7) ^ sub;
    const int64_t kb = k0 + lch * 16;
    // A k-chunk past K gets an offset above every in-range one (row * ld < 2^31).
    const uint32_t koff = kb < kbytes ? (uint32_t)kb : 0x80000000u;
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
        const int c = wave + 4 * i;
        const uint32_t off = (uint32_t)(c * 8 + sub) * ld + koff;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (H3Q_LDS void*)(dst + c * 1024), 16, off, 0, 0, 0);
    }
}

// Fragment of one 32-row MFMA operand for k-step s of a stage.
template <int OP>
__device__ __forceinline__ typename Mfma<OP>::frag_t read_frag(const H3Q_LDS uint8_t* tile, int row, int s, int g) {
    const H3Q_LDS uint8_t* base = tile + row * kBK;
    const int sw = row & 7;
    if constexpr (OP == kOpE4M3) {
        const int c0 = s * 4 + g * 2;
        v4i lo = *(const H3Q_LDS v4i*)(base + ((c0 ^ sw) << 4));
        v4i hi = *(const H3Q_LDS v4i*)(base + (((c0 + 1) ^ sw) << 4));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
        const int c = s * 2 + g;
        return *(const H3Q_LDS v4i*)(base + ((c ^ sw) << 4));
    }
}

template <int OP, int TM, int TN>
__device__ __forceinline__ void mma_stage(const H3Q_LDS uint8_t* sa, const H3Q_LDS uint8_t* sb, int wm0, int wn0,
                                          int lane, typename Mfma<OP>::acc_t (&acc)[TM][TN]) {
    constexpr int kSteps = kBK / Mfma<OP>::kStep;
    const int r = lane & 31, g = lane >> 5;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        typename Mfma<OP>::frag_t af[TM], bfr[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = read_frag<OP>(sa, wm0 + 32 * i + r, s, g);
#pragma unroll
        for (int j = 0; j < TN; ++j) bfr[j] = read_frag<OP>(sb, wn0 + 32 * j + r, s, g);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<OP>::run(af[i], bfr[j], acc[i][j]);
    }
}

// Logical tile for this workgroup.  Workgroups are dealt to the 8 XCDs round
// robin (XCD = blockIdx % 8); give each XCD a contiguous run of tiles so the
// tiles resident on one XCD share A and B rows in that XCD's L2.  Within the
// run, tiles go column-major in groups of kGroupM tile-rows.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kXcds = 8, kGroupM = 8;
    const int total = tiles_m * tiles_n;
    const int bid = blockIdx.x;
    const int q = total / kXcds, rem = total % kXcds;
    const int xcd = bid % kXcds, local = bid / kXcds;
    const int t = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
    const int per_group = kGroupM * tiles_n;
    const int group = t / per_group;
    const int first_m = group * kGroupM;
    const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int in_group = t - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

enum Epi : int { kEpiScaled = 0, kEpiI32 = 1, kEpiBF16 = 2 };

template <int OP, int BM, int BN, int EPI, bool LORA>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmArgs p, int tiles_m, int tiles_n) {
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int kStage = (BM + BN) * kBK;
    using acc_t = typename Mfma<OP>::acc_t;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_stage0[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_stage1[kStage];
    H3Q_LDS uint8_t* const lds0 = (H3Q_LDS uint8_t*)lds_stage0;
    H3Q_LDS uint8_t* const lds1 = (H3Q_LDS uint8_t*)lds_stage1;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int tm, tn;
    tile_coords(tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

    const int64_t kbytes = (OP == kOpBF16) ? p.k * 2 : p.k;
    const int64_t rows_a = (p.m - m0) < BM ? (p.m - m0) : BM;
    const int64_t rows_b = (p.n - n0) < BN ? (p.n - n0) : BN;
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc((const uint8_t*)p.a + m0 * p.lda, (uint32_t)(rows_a * p.lda));
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc((const uint8_t*)p.b + n0 * p.ldb, (uint32_t)(rows_b * p.ldb));

    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};

    const int64_t ktiles = (kbytes + kBK - 1) / kBK;
    load_tile<BM>(ra, lds0, (uint32_t)p.lda, 0, kbytes, wave, lane);
    load_tile<BN>(rb, lds0 + BM * kBK, (uint32_t)p.ldb, 0, kbytes, wave, lane);
    wait_vmcnt0();
    __syncthreads();
    for (int64_t kt = 0; kt < ktiles; ++kt) {
        H3Q_LDS uint8_t* cur = (kt & 1) ? lds1 : lds0;
        H3Q_LDS uint8_t* nxt = (kt & 1) ? lds0 : lds1;
        if (kt + 1 < ktiles) {
            load_tile<BM>(ra, nxt, (uint32_t)p.lda, (kt + 1) * kBK, kbytes, wave, lane);
            load_tile<BN>(rb, nxt + BM * kBK, (uint32_t)p.ldb, (kt + 1) * kBK, kbytes, wave, lane);
        }
        mma_stage<OP, TM, TN>(cur, cur + BM * kBK, wm0, wn0, lane, acc);
        wait_vmcnt0();
        __syncthreads();
    }

    // LoRA slab: t [BM, r] and lora_b [BN, r] (bf16, r <= 128) staged into the
    // two LDS stages, 64 rank elements (128 B) per stage.
    if constexpr (LORA) {
        const int64_t rbytes = p.lora_rank * 2;
        const __amdgpu_buffer_rsrc_t rt =
            make_rsrc((const uint8_t*)p.lora_t + m0 * p.ldt * 2, (uint32_t)(rows_a * p.ldt * 2));
        const __amdgpu_buffer_rsrc_t rl =
            make_rsrc((const uint8_t*)p.lora_b + n0 * p.ldlb * 2, (uint32_t)(rows_b * p.ldlb * 2));
        load_tile<BM>(rt, lds0, (uint32_t)(p.ldt * 2), 0, rbytes, wave, lane);
        load_tile<BN>(rl, lds0 + BM * kBK, (uint32_t)(p.ldlb * 2), 0, rbytes, wave, lane);
        load_tile<BM>(rt, lds1, (uint32_t)(p.ldt * 2), kBK, rbytes, wave, lane);
        load_tile<BN>(rl, lds1 + BM * kBK, (uint32_t)(p.ldlb * 2), kBK, rbytes, wave, lane);
        wait_vmcnt0();
        __syncthreads();
    }

    const int g = lane >> 5, c32 = lane & 31;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t col = n0 + wn0 + 32 * j + c32;
            const int64_t row_base = m0 + wm0 + 32 * i + 4 * g;
            if constexpr (EPI == kEpiI32) {
                int32_t* out = (int32_t*)p.out;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t row = row_base + 8 * (v >> 2) + (v & 3);
                    if (row < p.m && col < p.n) out[row * p.ldo + col] = acc[i][j][v];
                }
            } else if constexpr (EPI == kEpiBF16) {
                uint16_t* out = (uint16_t*)p.out;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t row = row_base + 8 * (v >> 2) + (v & 3);
                    if (row < p.m && col < p.n) out[row * p.ldo + col] = (uint16_t)f32_to_bf16_bits(acc[i][j][v]);
                }
            } else {
                v16f lora{};
                if constexpr (LORA) {
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        lora = Mfma<kOpBF16>::run(read_frag<kOpBF16>(lds0, wm0 + 32 * i + c32, s, g),
                                                  read_frag<kOpBF16>(lds0 + BM * kBK, wn0 + 32 * j + c32, s, g),
                                                  lora);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        lora = Mfma<kOpBF16>::run(read_frag<kOpBF16>(lds1, wm0 + 32 * i + c32, s, g),
                                                  read_frag<kOpBF16>(lds1 + BM * kBK, wn0 + 32 * j + c32, s, g),
                                                  lora);
                }
                const bool cin = col < p.n;
                const float sw = p.b_scale[p.b_scale_per_col ? (cin ? col : 0) : 0];
                const float bias = (p.bias && cin) ? bf16_lo(p.bias[col]) : 0.0f;
                uint16_t* out = (uint16_t*)p.out;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t row = row_base + 8 * (v >> 2) + (v & 3);
                    if (row < p.m && cin) {
                        const float sa = p.a_scale[p.a_scale_per_row ? row : 0];
                        const float t = __fmul_rn(sw, (float)acc[i][j][v]);
                        float y = p.bias ? __builtin_fmaf(sa, t, bias) : __fmul_rn(sa, t);
                        if constexpr (LORA) y = __builtin_fmaf(p.lora_scale, lora[v], y);
                        out[row * p.ldo + col] = (uint16_t)f32_to_bf16_bits(y);
                    }
                }
            }
        }
    }
}

template <int OP, int BM, int BN, int EPI, bool LORA>
static hipError_t launch(const GemmArgs& a, hipStream_t st) {
    const int tiles_m = (int)((a.m + BM - 1) / BM), tiles_n = (int)((a.n + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_kernel<OP, BM, BN, EPI, LORA>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st,
                       a, tiles_m, tiles_n);
    return hipGetLastError();
}

hipError_t launch_gemm(int kind, bool raw_i32, const GemmArgs& a, hipStream_t st) {
    const bool lora = a.lora_t != nullptr;
    if (kind == kOpE4M3) {
        return lora ? launch<kOpE4M3, 256, 256, kEpiScaled, true>(a, st)
                    : launch<kOpE4M3, 256, 256, kEpiScaled, false>(a, st);
    }
    if (kind == kOpInt8) {
        if (raw_i32) return launch<kOpInt8, 256, 256, kEpiI32, false>(a, st);
        return lora ? launch<kOpInt8, 256, 256, kEpiScaled, true>(a, st)
                    : launch<kOpInt8, 256, 256, kEpiScaled, false>(a, st);
    }
    return launch<kOpBF16, 128, 128, kEpiBF16, false>(a, st);
}

}  // namespace h3q
