// Scaled FP8 / INT8 GEMM (and the bf16 LoRA down-projection) on gfx950 MFMA.
//
//   out[m, n] = epilogue( sum_k A[m, k] * B[n, k] )
//
// A and B are both K-contiguous ("TN": activations [M, K] and nn.Linear
// weights [N, K]).  A block tile BM x BN is split over WAVES_M x WAVES_N
// wavefronts, each owning a (BM/WAVES_M) x (BN/WAVES_N) accumulator block of
// 32 x 32 MFMA tiles:
//   e4m3  v_mfma_f32_32x32x64_f8f6f4   (32 code bytes per lane per operand)
//   int8  v_mfma_i32_32x32x32_i8       (16 bytes per lane)
//   bf16  v_mfma_f32_32x32x16_bf16     (16 bytes per lane)
//
// Pipeline.  K advances in tiles of BK bytes.  Each operand tile (rows x BK)
// is copied HBM -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging) into
// a ring of STAGES LDS buffers; STAGES - 1 tiles are in flight while the
// MFMAs consume the oldest.  One workgroup barrier per k-tile both publishes
// the tile that just landed and frees the buffer the next copy overwrites.
//
// LDS layout.  A row of a stage holds BK / 16 chunks of 16 bytes; logical
// chunk c of row r sits at physical chunk c ^ f(r), f(r) = (r / (128 / BK))
// mod (BK / 16), so the lanes of one ds_read_b128 phase (consecutive rows,
// same logical chunk) spread over distinct bank groups.  One wave copy
// instruction fills 1 KiB: lane L lands at byte 16 L of it, so it fetches the
// logical chunk that the layout assigns to that position.
//
// Tails.  Rows beyond M / N and chunks beyond K are fetched with an
// out-of-range buffer offset, which the hardware returns as zeros.
//
// Epilogue (per 32 x 32 tile, in registers):
//   e4m3 / int8: v = s_a[m] * (s_w[n] * float(acc)) [fma(s_a, ., bias[n])]
//                [+ lora_scale * (t[m, :] . lora_b[n, :])  (bf16 MFMA slab)]
//                -> bf16 round-to-nearest-even
//   raw int32:   acc
//   bf16 GEMM:   bf16(acc)
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"
#include "gemm_tiles.hpp"

namespace h3q {

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

// OCC_ = waves per SIMD the register budget is sized for (1: one 4-wave
// workgroup per CU with 512 registers per lane; 2: two workgroups per CU or
// one 8-wave workgroup).
template <int BM_, int BN_, int BK_, int STAGES_, int WAVES_M_, int WAVES_N_, int OCC_ = 1>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, STAGES = STAGES_, OCC = OCC_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, NWAVES = WAVES_M * WAVES_N;
    static constexpr int NT = 64 * NWAVES;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N, TM = WM / 32, TN = WN / 32;
    static constexpr int CH = BK / 16;           // 16-byte chunks per row
    static constexpr int ROWS_PER_KB = 1024 / BK;
    static constexpr int STAGE_BYTES = (BM + BN) * BK;
    static constexpr int LOADS_A = BM * BK / 1024 / NWAVES;  // copy instructions per wave per stage
    static constexpr int LOADS_B = BN * BK / 1024 / NWAVES;
    static constexpr int LOADS = LOADS_A + LOADS_B;
    static_assert(BK == 64 || BK == 128, "BK");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile");
    static_assert((BM * BK / 1024) % NWAVES == 0 && (BN * BK / 1024) % NWAVES == 0, "copy split");
    static_assert(STAGES >= 2 && STAGES * STAGE_BYTES * (OCC * 4 / NWAVES > 0 ? OCC * 4 / NWAVES : 1) <= 160 * 1024, "LDS");
    static_assert(LOADS * (STAGES - 2) < 64, "vmcnt");
    // Physical chunk = logical chunk ^ swz(row).  gfx950's LDS serves 256
    // bytes per clock, i.e. 16 lanes of a ds_read_b128 at once; those 16
    // lanes read 16 consecutive rows at the same logical chunk, covering
    // 16 * BK bytes, so their 16-byte slots (row * BK + 16 * phys) mod 256
    // must all differ.  For BK = 128 rows pair up in a 256-byte window and
    // the eight rows of equal parity need distinct chunks: swz = (r ^ r>>3)
    // mod 8.  For BK = 64 four rows share a window and rows r, r+4, r+8, r+12
    // need distinct chunks: swz = (r>>1 ^ r>>3) mod 2 + 2 ((r>>2) mod 2).  Both
    // also keep any 8 consecutive rows conflict-free.
    static __device__ __forceinline__ int swz(int r) {
        if constexpr (BK == 128) return (r ^ (r >> 3)) & 7;
        return (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2);
    }
};

// Copy rows [0, ROWS) x bytes [k0, k0 + BK) of an operand into an LDS stage.
template <class T, int ROWS>
__device__ __forceinline__ void load_tile(const CopySrc& rsrc, H3Q_LDS uint8_t* dst, uint32_t ld,
                                          int64_t k0, int64_t kbytes, int wave, int lane) {
    const int sub = lane / T::CH;  // row inside the 1 KiB copy
#pragma unroll
    for (int i = 0; i < ROWS * T::BK / 1024 / T::NWAVES; ++i) {
        const int c = wave + T::NWAVES * i;
        const int row = c * T::ROWS_PER_KB + sub;
        const int64_t kb = k0 + ((lane % T::CH) ^ T::swz(row)) * 16;  // logical chunk this lane fetches
        // A chunk past K gets an offset above every in-range one (row * ld < 2^31).
        const uint32_t off = kb < kbytes ? (uint32_t)row * ld + (uint32_t)kb : 0x80000000u;
        copy16(rsrc, (uint32_t)(uintptr_t)(dst + c * 1024), off);
    }
}

// MFMA operand fragment of one 32-row block for k-step s of a stage.
template <class T, int OP>
__device__ __forceinline__ typename Mfma<OP>::frag_t read_frag(const H3Q_LDS uint8_t* tile, int row, int s, int g) {
    const H3Q_LDS uint8_t* base = tile + row * T::BK;
    const int sw = T::swz(row);
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

// Tiled operand (16-row x 128-byte blocks of 2 KiB in MFMA fragment order,
// see code_offset in act_quant.hip): stage kt of a BN-row tile is BN / 16
// blocks, each two 1 KiB halves, copied contiguously (block b, half h at LDS
// byte (2 b + h) * 1024).  Rows past N are whole blocks past the descriptor.
template <class T, int ROWS>
__device__ __forceinline__ void load_tile_tiled(const CopySrc& rsrc, H3Q_LDS uint8_t* dst, int64_t steps, int kt,
                                                int64_t nblk, int wave, int lane) {
    static_assert(T::BK == 128, "tiled operands come in 128-byte k-steps");
#pragma unroll
    for (int i = 0; i < ROWS * 128 / 1024 / T::NWAVES; ++i) {
        const int c = wave + T::NWAVES * i;
        const int blk = c >> 1;
        const uint32_t off = blk < nblk ? (uint32_t)(((int64_t)blk * steps + kt) * 2048 + (c & 1) * 1024 + 16 * lane)
                                        : 0x80000000u;
        copy16(rsrc, (uint32_t)(uintptr_t)(dst + c * 1024), off);
    }
}

// Fragment of row `row` for k-step s from a tiled stage: its bytes k = kStep * s
// + (fragment bytes) * g live in block row / 16, lane slot row % 16 + 16 q of
// the 128-byte step (q = k / 32), halves 1 KiB apart.  Sixteen consecutive
// rows read 16 consecutive 16-byte slots: no bank conflicts.
template <int OP>
__device__ __forceinline__ typename Mfma<OP>::frag_t read_frag_tiled(const H3Q_LDS uint8_t* tile, int row, int s,
                                                                     int g) {
    const H3Q_LDS uint8_t* blk = tile + (row >> 4) * 2048;
    if constexpr (OP == kOpE4M3) {
        const int slot = (row & 15) + 16 * (2 * s + g);
        const v4i lo = *(const H3Q_LDS v4i*)(blk + 16 * slot);
        const v4i hi = *(const H3Q_LDS v4i*)(blk + 1024 + 16 * slot);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
        const int slot = (row & 15) + 16 * s;
        return *(const H3Q_LDS v4i*)(blk + g * 1024 + 16 * slot);
    }
}

// One stage of MFMAs.  The weight fragment is the MFMA's A operand and the
// activation fragment its B operand, so accumulator tile acc[i][j] holds
// out^T: lane L owns output row m = 32 i + L % 32 and, in accumulator slot v,
// column n = 32 j + 8 (v / 4) + 4 (L / 32) + v % 4 -- four consecutive
// columns per slot group, which the epilogue writes as one 8-byte store.
template <class T, int OP, bool TB>
__device__ __forceinline__ void mma_stage(const H3Q_LDS uint8_t* sa, const H3Q_LDS uint8_t* sb, int wm0, int wn0,
                                          int lane, typename Mfma<OP>::acc_t (&acc)[T::TM][T::TN]) {
    constexpr int kSteps = T::BK / Mfma<OP>::kStep;
    const int r = lane & 31, g = lane >> 5;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        typename Mfma<OP>::frag_t af[T::TM], bfr[T::TN];
#pragma unroll
        for (int i = 0; i < T::TM; ++i) af[i] = read_frag<T, OP>(sa, wm0 + 32 * i + r, s, g);
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
            bfr[j] = TB ? read_frag_tiled<OP>(sb, wn0 + 32 * j + r, s, g) : read_frag<T, OP>(sb, wn0 + 32 * j + r, s, g);
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int j = 0; j < T::TN; ++j) acc[i][j] = Mfma<OP>::run(bfr[j], af[i], acc[i][j]);
    }
}

// kEpiScaledF16: the scaled epilogue with binary16 bias and output.
enum Epi : int { kEpiScaled = 0, kEpiI32 = 1, kEpiBF16 = 2, kEpiScaledF16 = 3, kEpiF32 = 4 };

// Wait until the oldest `pending + 1` copy stages of this wave have landed,
// leaving `pending` younger stages in flight (only used while draining).
template <class T>
__device__ __forceinline__ void wait_stage(int pending) {
    if constexpr (T::STAGES >= 4) {
        if (pending >= 2) { wait_vmcnt<2 * T::LOADS>(); return; }
    }
    if constexpr (T::STAGES >= 3) {
        if (pending >= 1) { wait_vmcnt<T::LOADS>(); return; }
    }
    wait_vmcnt<0>();
}

// Kernel variants.  The epilogue is fully unrolled (all accumulators live in
// registers), so every choice inside it is a template parameter rather than a
// branch: VEC (4 columns per store; needs ldo % 4 == 0, n % 4 == 0 and a
// 16-byte aligned output) and BIAS.  The scalar-store variant (VEC = false)
// takes the bias from a runtime check.
template <class T, int OP, int EPI, bool LORA, bool VEC, bool BIAS, bool TB>
__global__ __launch_bounds__(T::NT, T::OCC) void gemm_kernel(GemmArgs p, int tiles_m, int tiles_n) {
    constexpr int BM = T::BM, BN = T::BN, BK = T::BK, S = T::STAGES, TM = T::TM, TN = T::TN;
    using acc_t = typename Mfma<OP>::acc_t;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_ring[S * T::STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) float lds_sw[BN];     // this block's per-column weight scales
    __shared__ __attribute__((aligned(16))) uint16_t lds_bias[BN];  // and bias (bf16 bits)
    H3Q_LDS uint8_t* const lds = (H3Q_LDS uint8_t*)lds_ring;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 5, c32 = lane & 31;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int wm0 = (wave / T::WAVES_N) * T::WM, wn0 = (wave % T::WAVES_N) * T::WN;

    const int64_t kbytes = (OP == kOpBF16) ? p.k * 2 : p.k;
    const int64_t rows_a = (p.m - m0) < BM ? (p.m - m0) : BM;
    const int64_t rows_b = (p.n - n0) < BN ? (p.n - n0) : BN;
    const CopySrc ra((const uint8_t*)p.a + m0 * p.lda, (uint32_t)(rows_a * p.lda));
    const int64_t steps = kbytes / 128;                    // tiled B: 128-byte k-steps
    const int64_t nblk = (rows_b + 15) / 16;               // tiled B: 16-row blocks in this tile
    const CopySrc rb(TB ? (const uint8_t*)p.b + (n0 / 16) * steps * 2048 : (const uint8_t*)p.b + n0 * p.ldb,
                     TB ? (uint32_t)(nblk * steps * 2048) : (uint32_t)(rows_b * p.ldb));

    // Scales are fetched before the main loop so their latency hides behind
    // it: each lane's row scales in registers, the block's column scales and
    // bias in LDS (published by the first ring barrier).
    constexpr bool kScaled = EPI == kEpiScaled || EPI == kEpiScaledF16;
    constexpr bool kF16 = EPI == kEpiScaledF16;
    float sa_reg[TM];
    if constexpr (kScaled) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t m = m0 + wm0 + 32 * i + c32;
            sa_reg[i] = m < p.m ? p.a_scale[p.a_scale_per_row ? m : 0] : 0.0f;
        }
        for (int c = threadIdx.x; c < BN; c += T::NT) {
            const int64_t n = n0 + c;
            lds_sw[c] = n < p.n ? p.b_scale[p.b_scale_per_col ? n : 0] : 0.0f;
            if (BIAS || !VEC) lds_bias[c] = (p.bias && n < p.n) ? p.bias[n] : (uint16_t)0;
        }
    }

    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};

    // Main loop.  The steady state always has S - 2 younger stages in flight
    // behind the one it waits for, so its body is branch-free; the last
    // S - 1 k-tiles drain the ring.
    // kEpiF32: blockIdx.y takes k-tiles kt0 .. kt0 + p.kt_split - 1 (a slice
    // of a split over K) and stores its binary32 partial sums.
    const int ktiles_all = (int)((kbytes + BK - 1) / BK);
    const int kt0 = EPI == kEpiF32 ? (int)(blockIdx.y * p.kt_split) : 0;
    const int ktiles = EPI == kEpiF32 ? (ktiles_all - kt0 < (int)p.kt_split ? ktiles_all - kt0 : (int)p.kt_split)
                                      : ktiles_all;
    auto issue = [&](int kt, int buf) {
        H3Q_LDS uint8_t* dst = lds + buf * T::STAGE_BYTES;
        load_tile<T, BM>(ra, dst, (uint32_t)p.lda, (int64_t)(kt0 + kt) * BK, kbytes, wave, lane);
        if constexpr (TB) load_tile_tiled<T, BN>(rb, dst + BM * BK, steps, kt, nblk, wave, lane);
        else load_tile<T, BN>(rb, dst + BM * BK, (uint32_t)p.ldb, (int64_t)(kt0 + kt) * BK, kbytes, wave, lane);
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < ktiles) issue(s, s);
    int rd = 0, wr = S - 1, kt = 0;
    for (; kt + S - 1 < ktiles; ++kt) {
        wait_vmcnt<(S - 2) * T::LOADS>();
        ring_barrier();
        issue(kt + S - 1, wr);
        const H3Q_LDS uint8_t* cur = lds + rd * T::STAGE_BYTES;
        mma_stage<T, OP, TB>(cur, cur + BM * BK, wm0, wn0, lane, acc);
        rd = rd + 1 == S ? 0 : rd + 1;
        wr = wr + 1 == S ? 0 : wr + 1;
    }
    for (; kt < ktiles; ++kt) {
        wait_stage<T>(ktiles - 1 - kt);
        ring_barrier();
        const H3Q_LDS uint8_t* cur = lds + rd * T::STAGE_BYTES;
        mma_stage<T, OP, TB>(cur, cur + BM * BK, wm0, wn0, lane, acc);
        rd = rd + 1 == S ? 0 : rd + 1;
    }

    // LoRA slab: t [BM, r] and lora_b [BN, r] (bf16, r <= 128 -> 256 bytes per
    // row) staged into the first 256 / BK ring buffers.
    constexpr int kLoraTiles = 256 / BK;
    if constexpr (LORA) {
        static_assert(kLoraTiles <= S, "LoRA slab needs 256 bytes of K per row across the ring");
        __syncthreads();
        const int64_t rbytes = p.lora_rank * 2;
        const CopySrc rt((const uint8_t*)p.lora_t + m0 * p.ldt * 2, (uint32_t)(rows_a * p.ldt * 2));
        const CopySrc rl((const uint8_t*)p.lora_b + n0 * p.ldlb * 2, (uint32_t)(rows_b * p.ldlb * 2));
#pragma unroll
        for (int t = 0; t < kLoraTiles; ++t) {
            H3Q_LDS uint8_t* dst = lds + t * T::STAGE_BYTES;
            load_tile<T, BM>(rt, dst, (uint32_t)(p.ldt * 2), t * BK, rbytes, wave, lane);
            load_tile<T, BN>(rl, dst + BM * BK, (uint32_t)(p.ldlb * 2), t * BK, rbytes, wave, lane);
        }
        wait_vmcnt<0>();
        __syncthreads();
    }

    // Epilogue.  Stores go through a buffer resource over this block's output
    // rows, so rows past M fall outside it and are dropped by the hardware;
    // a column group past N is given an out-of-range offset.
    constexpr uint32_t kEs = EPI == kEpiI32 || EPI == kEpiF32 ? 4 : 2;
    constexpr uint32_t kDrop = 0xFFFFFFF0u;
    // kEpiF32: slice blockIdx.y's partial is the [m, ldo] binary32 block y of out.
    const int64_t slice_row0 = EPI == kEpiF32 ? (int64_t)blockIdx.y * p.m : 0;
    const __amdgpu_buffer_rsrc_t ro =
        make_rsrc((uint8_t*)p.out + (slice_row0 + m0) * p.ldo * kEs, (uint32_t)(rows_a * p.ldo * kEs));
    const H3Q_LDS float* sw_l = (const H3Q_LDS float*)lds_sw;
    const H3Q_LDS uint16_t* bias_l = (const H3Q_LDS uint16_t*)lds_bias;
    const bool has_bias = VEC ? BIAS : p.bias != nullptr;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint32_t row_off = (uint32_t)(wm0 + 32 * i + c32) * (uint32_t)p.ldo * kEs;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            // Keep each output tile's LDS reads and MFMAs from being hoisted
            // into earlier tiles (register pressure: all accumulators are live).
            __builtin_amdgcn_sched_barrier(0);
            v16f lora{};
            if constexpr (LORA) {
#pragma unroll
                for (int t = 0; t < kLoraTiles; ++t) {
                    const H3Q_LDS uint8_t* st = lds + t * T::STAGE_BYTES;
#pragma unroll
                    for (int s = 0; s < BK / 32; ++s)
                        lora = Mfma<kOpBF16>::run(read_frag<T, kOpBF16>(st + BM * BK, wn0 + 32 * j + c32, s, g),
                                                  read_frag<T, kOpBF16>(st, wm0 + 32 * i + c32, s, g), lora);
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int nl = wn0 + 32 * j + 8 * q + 4 * g;  // first of this slot group's 4 columns
                const int64_t n = n0 + nl;
                if constexpr (EPI == kEpiI32 || EPI == kEpiF32) {
                    v4i d;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const auto v = acc[i][j][4 * q + e];
                        if constexpr (EPI == kEpiF32) d[e] = __float_as_int(v);
                        else d[e] = v;
                    }
                    if constexpr (VEC) {
                        const uint32_t off = n < p.n ? row_off + (uint32_t)n * kEs : kDrop;
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, d), ro, off, 0, 0);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t off = n + e < p.n ? row_off + (uint32_t)(n + e) * kEs : kDrop;
                            __builtin_amdgcn_raw_buffer_store_b32((uint32_t)d[e], ro, off, 0, 0);
                        }
                    }
                } else {
                    float y[4];
                    if constexpr (EPI == kEpiBF16) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) y[e] = acc[i][j][4 * q + e];
                    } else {
                        const v4f sw4 = *(const H3Q_LDS v4f*)(sw_l + nl);
                        v2u b4 = {0u, 0u};
                        if (BIAS || !VEC) b4 = *(const H3Q_LDS v2u*)(bias_l + nl);
                        const float bias[4] = {out_lo(b4[0], kF16), out_hi(b4[0], kF16), out_lo(b4[1], kF16),
                                               out_hi(b4[1], kF16)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float t = __fmul_rn(sw4[e], (float)acc[i][j][4 * q + e]);
                            float v = has_bias ? __builtin_fmaf(sa_reg[i], t, bias[e]) : __fmul_rn(sa_reg[i], t);
                            if constexpr (LORA) v = __builtin_fmaf(p.lora_scale, lora[4 * q + e], v);
                            y[e] = v;
                        }
                    }
                    const uint32_t w0 = pack_out2(y[0], y[1], kF16), w1 = pack_out2(y[2], y[3], kF16);
                    if constexpr (VEC) {
                        const uint32_t off = n < p.n ? row_off + (uint32_t)n * kEs : kDrop;
                        __builtin_amdgcn_raw_buffer_store_b64(v2u{w0, w1}, ro, off, 0, 0);
                    } else {
                        const uint16_t h[4] = {(uint16_t)w0, (uint16_t)(w0 >> 16), (uint16_t)w1, (uint16_t)(w1 >> 16)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t off = n + e < p.n ? row_off + (uint32_t)(n + e) * kEs : kDrop;
                            __builtin_amdgcn_raw_buffer_store_b16(h[e], ro, off, 0, 0);
                        }
                    }
                }
            }
        }
    }
}

// Persistent scaled GEMM (e4m3 / int8 -> bf16, optional bias, no LoRA, 4-column
// stores).  A grid of at most one workgroup per CU walks the output tiles
// blockIdx.x, blockIdx.x + gridDim.x, ... with one continuous 2-stage copy
// ring: the last k-tile of a tile issues the first stage of the next one, so
// that copy is in flight during the last MFMAs and the epilogue, and no
// workgroup is relaunched between tiles (on MI355X a 16-wave workgroup with
// 128 KiB of LDS takes about 7 us from the end of one to the start of the next
// on the same CU, measured with s_memrealtime).  The tile's per-row /
// per-column scales and bias are copied into LDS with its first stage,
// double-buffered by tile parity; a per-tensor scale is read once.
// Arithmetic, k order and rounding are those of gemm_kernel: both produce the
// same bits.
template <class T, int OP, bool BIAS, bool TB>
__global__ __launch_bounds__(T::NT, T::OCC) void gemm_persistent_kernel(GemmArgs p, int tiles_m, int tiles_n) {
    constexpr int BM = T::BM, BN = T::BN, BK = T::BK, TM = T::TM, TN = T::TN;
    static_assert(BM == 256 && BN == 256, "one 1 KiB copy per scale vector");
    static_assert(T::STAGES == 2, "two-stage ring");
    static_assert(OP != kOpBF16, "codes only");
    using acc_t = typename Mfma<OP>::acc_t;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_ring[2 * T::STAGE_BYTES];
    // Per tile parity: row scales [BM] f32 | column scales [BN] f32 | bias [BN] bf16.
    __shared__ __attribute__((aligned(1024))) uint8_t lds_ep[2 * 3 * 1024];
    H3Q_LDS uint8_t* const lds = (H3Q_LDS uint8_t*)lds_ring;
    H3Q_LDS uint8_t* const ep = (H3Q_LDS uint8_t*)lds_ep;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm0 = (wave / T::WAVES_N) * T::WM, wn0 = (wave % T::WAVES_N) * T::WN;
    const int ktiles = (int)((p.k + BK - 1) / BK);
    const int ntiles = (tiles_m * tiles_n - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const bool row_scales = p.a_scale_per_row != 0, col_scales = p.b_scale_per_col != 0;
    // A per-tensor scale fills its LDS vector (both parities) once; per-row /
    // per-column vectors are copied per tile.
    if (!row_scales || !col_scales) {
        const float sa0 = row_scales ? 0.0f : p.a_scale[0], sw0 = col_scales ? 0.0f : p.b_scale[0];
        for (int c = threadIdx.x; c < 2 * 256; c += T::NT) {
            H3Q_LDS float* e = (H3Q_LDS float*)(ep + (c >> 8) * 3072);
            if (!row_scales) e[c & 255] = sa0;
            if (!col_scales) e[256 + (c & 255)] = sw0;
        }
    }

    // Origin and extent of local tile j.
    struct TileSrc {
        int m0, n0, rows, cols;
    };
    auto tile_src = [&](int j) {
        int tm, tn;
        tile_coords((int)blockIdx.x + j * (int)gridDim.x, tiles_m, tiles_n, tm, tn);
        TileSrc t;
        t.m0 = tm * BM;
        t.n0 = tn * BN;
        t.rows = (int)(p.m - t.m0 < BM ? p.m - t.m0 : BM);
        t.cols = (int)(p.n - t.n0 < BN ? p.n - t.n0 : BN);
        return t;
    };
    const int64_t steps = p.k / 128;  // tiled B: 128-byte k-steps
    auto a_src = [&](const TileSrc& t) {
        return CopySrc((const uint8_t*)p.a + (int64_t)t.m0 * p.lda, (uint32_t)((int64_t)t.rows * p.lda));
    };
    auto b_src = [&](const TileSrc& t) {
        if constexpr (TB)
            return CopySrc((const uint8_t*)p.b + (int64_t)(t.n0 / 16) * steps * 2048,
                           (uint32_t)((t.cols + 15) / 16 * steps * 2048));
        else
            return CopySrc((const uint8_t*)p.b + (int64_t)t.n0 * p.ldb, (uint32_t)((int64_t)t.cols * p.ldb));
    };
    // The epilogue vectors of tile j, issued ahead of its first stage so the
    // wait for that stage covers them.  Past the operand ends copies read zeros.
    auto issue_vectors = [&](const TileSrc& t, int j, int ln) {
        H3Q_LDS uint8_t* e = ep + (j & 1) * 3072;
        if (wave == 0 && row_scales)
            copy16(CopySrc(p.a_scale + t.m0, (uint32_t)t.rows * 4u), (uint32_t)(uintptr_t)e, 16u * ln);
        if (wave == 1 && col_scales)
            copy16(CopySrc(p.b_scale + t.n0, (uint32_t)t.cols * 4u), (uint32_t)(uintptr_t)(e + 1024), 16u * ln);
        if (BIAS && wave == 2)
            copy16(CopySrc(p.bias + t.n0, (uint32_t)t.cols * 2u), (uint32_t)(uintptr_t)(e + 2048),
                   ln < 32 ? 16u * ln : 0x80000000u);
    };
    auto issue_stage = [&](const CopySrc& ra, const CopySrc& rb, int nblk, int kt, int buf, int ln) {
        H3Q_LDS uint8_t* dst = lds + buf * T::STAGE_BYTES;
        load_tile<T, BM>(ra, dst, (uint32_t)p.lda, (int64_t)kt * BK, p.k, wave, ln);
        if constexpr (TB) load_tile_tiled<T, BN>(rb, dst + BM * BK, steps, kt, nblk, wave, ln);
        else load_tile<T, BN>(rb, dst + BM * BK, (uint32_t)p.ldb, (int64_t)kt * BK, p.k, wave, ln);
    };

    {
        const TileSrc t = tile_src(0);
        issue_vectors(t, 0, lane);
        issue_stage(a_src(t), b_src(t), (t.cols + 15) / 16, 0, 0, lane);
    }
    int rd = 0;
    for (int j = 0; j < ntiles; ++j) {
        const int lane = opaque_lane();
        CopySrc ra(nullptr, 0), rb(nullptr, 0);
        int nblk;
        {
            const TileSrc t = tile_src(j);
            ra = a_src(t);
            rb = b_src(t);
            nblk = (t.cols + 15) / 16;
        }
        acc_t acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int jj = 0; jj < TN; ++jj) acc[i][jj] = acc_t{};
        for (int kt = 0; kt < ktiles; ++kt) {
            // Everything this wave issued has landed (the copies of this
            // stage, and the previous epilogue's stores); the barrier makes
            // every wave's copies visible and frees the other buffer.
            wait_vmcnt<0>();
            ring_barrier();
            if (kt + 1 < ktiles) {
                issue_stage(ra, rb, nblk, kt + 1, rd ^ 1, lane);
            } else if (j + 1 < ntiles) {
                const TileSrc t = tile_src(j + 1);
                issue_vectors(t, j + 1, lane);
                issue_stage(a_src(t), b_src(t), (t.cols + 15) / 16, 0, rd ^ 1, lane);
            }
            const H3Q_LDS uint8_t* st = lds + rd * T::STAGE_BYTES;
            mma_stage<T, OP, TB>(st, st + BM * BK, wm0, wn0, lane, acc);
            rd ^= 1;
        }

        // Epilogue: v = s_a[m] * (s_w[n] * float(acc)) [fma with bias[n]] ->
        // bf16, 4 columns per 8-byte store through a buffer resource over the
        // tile's rows (rows past M are dropped by the hardware; a column
        // group past N gets an out-of-range offset).
        {
            const TileSrc cur = tile_src(j);
            const int g = lane >> 5, c32 = lane & 31;
            const H3Q_LDS uint8_t* e = ep + (j & 1) * 3072;
            const H3Q_LDS float* sa_l = (const H3Q_LDS float*)e;
            const H3Q_LDS float* sw_l = (const H3Q_LDS float*)(e + 1024);
            const H3Q_LDS uint16_t* bias_l = (const H3Q_LDS uint16_t*)(e + 2048);
            const __amdgpu_buffer_rsrc_t ro =
                make_rsrc((uint8_t*)p.out + (int64_t)cur.m0 * p.ldo * 2, (uint32_t)((int64_t)cur.rows * p.ldo * 2));
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int ml = wm0 + 32 * i + c32;
                const float sa = sa_l[ml];
                const uint32_t row_off = (uint32_t)ml * (uint32_t)p.ldo * 2u;
#pragma unroll
                for (int jj = 0; jj < TN; ++jj) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int nl = wn0 + 32 * jj + 8 * q + 4 * g;
                        const v4f sw4 = *(const H3Q_LDS v4f*)(sw_l + nl);
                        float y[4];
                        if constexpr (BIAS) {
                            const v2u b4 = *(const H3Q_LDS v2u*)(bias_l + nl);
                            const float bias[4] = {bf16_lo(b4[0]), bf16_hi(b4[0]), bf16_lo(b4[1]), bf16_hi(b4[1])};
#pragma unroll
                            for (int x = 0; x < 4; ++x)
                                y[x] = __builtin_fmaf(sa, __fmul_rn(sw4[x], (float)acc[i][jj][4 * q + x]), bias[x]);
                        } else {
#pragma unroll
                            for (int x = 0; x < 4; ++x) y[x] = __fmul_rn(sa, __fmul_rn(sw4[x], (float)acc[i][jj][4 * q + x]));
                        }
                        const uint32_t off = nl < cur.cols ? row_off + (uint32_t)(cur.n0 + nl) * 2u : 0xFFFFFFF0u;
                        __builtin_amdgcn_raw_buffer_store_b64(v2u{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])},
                                                              ro, off, 0, 0);
                    }
                }
            }
        }
    }
}

template <class T, int OP, int EPI, bool LORA, bool VEC, bool BIAS>
hipError_t launch_tile(const GemmArgs& a, hipStream_t st) {
    const int tiles_m = (int)((a.m + T::BM - 1) / T::BM), tiles_n = (int)((a.n + T::BN - 1) / T::BN);
    const dim3 grid((unsigned)(tiles_m * tiles_n));
    if constexpr (OP != kOpBF16 && T::BK == 128) {
        if (a.b_tiled) {
            hipLaunchKernelGGL((gemm_kernel<T, OP, EPI, LORA, VEC, BIAS, true>), grid, dim3(T::NT), 0, st, a, tiles_m,
                               tiles_n);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemm_kernel<T, OP, EPI, LORA, VEC, BIAS, false>), grid, dim3(T::NT), 0, st, a, tiles_m,
                       tiles_n);
    return hipGetLastError();
}

template <class T, int OP, bool BIAS>
hipError_t launch_persistent(const GemmArgs& a, hipStream_t st) {
    const int tiles_m = (int)((a.m + T::BM - 1) / T::BM), tiles_n = (int)((a.n + T::BN - 1) / T::BN);
    const dim3 grid((unsigned)persistent_grid(tiles_m * tiles_n));
    if (a.b_tiled)
        hipLaunchKernelGGL((gemm_persistent_kernel<T, OP, BIAS, true>), grid, dim3(T::NT), 0, st, a, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((gemm_persistent_kernel<T, OP, BIAS, false>), grid, dim3(T::NT), 0, st, a, tiles_m, tiles_n);
    return hipGetLastError();
}

// Selects the kernel and epilogue variant for a scaled GEMM.  The persistent
// kernel needs 4-column stores, no LoRA and at least STAGES k-tiles (its
// epilogue vectors are double-buffered across that many stages).
template <class T, int OP, bool LORA>
hipError_t launch_scaled(const GemmArgs& a, hipStream_t st) {
    if constexpr (!LORA) {
        // binary16 output (no LoRA): the tile kernel's F16 epilogue
        if (a.out_f16) {
            if (!a.out_vec) return launch_tile<T, OP, kEpiScaledF16, false, false, false>(a, st);
            return a.bias ? launch_tile<T, OP, kEpiScaledF16, false, true, true>(a, st)
                          : launch_tile<T, OP, kEpiScaledF16, false, true, false>(a, st);
        }
    }
    if constexpr (!LORA && T::BM == 256 && T::BN == 256 && T::BK == 128) {
        if (a.out_vec && (a.k + T::BK - 1) / T::BK >= T::STAGES)
            return a.bias ? launch_persistent<T, OP, true>(a, st) : launch_persistent<T, OP, false>(a, st);
    }
    if (!a.out_vec) return launch_tile<T, OP, kEpiScaled, LORA, false, false>(a, st);
    return a.bias ? launch_tile<T, OP, kEpiScaled, LORA, true, true>(a, st)
                  : launch_tile<T, OP, kEpiScaled, LORA, true, false>(a, st);
}

// Large-GEMM configuration: 256 x 256 block, 128-byte k-tiles, 2-deep ring
// (128 KiB of LDS), sixteen waves (4 x 4) of 64 x 64, four per SIMD.  The
// main loop is bound by the LDS-copy round trip of each 64 KiB stage, and
// sixteen waves issue the copies faster than eight (measured on MI355X at
// M=8192, N=15360, K=5120: 493 us vs 514 us with tiled weights).
using TileBig = Tile<256, 256, 128, 2, 4, 4, 4>;
// With the LoRA epilogue (an extra bf16 MFMA slab per output tile) the
// sixteen-wave register budget of 128 spills, so LoRA calls use eight waves
// (2 x 4) of 128 x 64 with 256 registers each.
using TileBigLora = Tile<256, 256, 128, 2, 2, 4, 2>;
// LoRA down-projection (N = rank <= 128): 128 x 128 blocks, bf16, 128-byte
// k-tiles in a 4-deep ring (128 KiB).  The call streams X once from HBM;
// measured on MI355X at M = 24576, r = 128: K = 13824 164 us and K = 5120
// 58 us, against 197 us and 67 us with 64-byte k-tiles.
using TileLora = Tile<128, 128, 128, 4, 2, 2>;
// Up to 256 x 96 rows the down-projection takes 96-row blocks (four waves of
// 96 x 32, a 5-deep ring of 28 KiB stages), so that up to 256 workgroups
// share the stream instead of M / 128 (M = 24576, same box, alternating:
// K = 5120 60.4-61.5 us against 65.5-66.1; K = 13824 181-188 against
// 185-186, no change).
using TileLora96 = Tile<96, 128, 128, 5, 1, 4>;

// Sum of the S binary32 partials of a split LoRA down-projection in slice
// order, rounded once to bf16: thread (row, 4-column group).
__global__ __launch_bounds__(256) void lora_down_reduce_kernel(const float* __restrict__ partial, int slices,
                                                               int64_t m, int rank, uint16_t* __restrict__ t,
                                                               int64_t ldt) {
    const int groups = rank / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= m * groups) return;
    const int64_t row = idx / groups;
    const int col = (int)(idx % groups) * 4;
    const v4f* src = reinterpret_cast<const v4f*>(partial + row * rank + col);
    const int64_t stride = m * rank / 4;  // one slice, in v4f
    v4f sum = src[0];
    for (int s = 1; s < slices; ++s) {
        const v4f v = src[s * stride];
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[e] = sum[e] + v[e];
    }
    *reinterpret_cast<v2u*>(t + row * ldt + col) = v2u{pack_out2(sum[0], sum[1], false), pack_out2(sum[2], sum[3], false)};
}

namespace {

// Slices of the split (1: no split): with fewer than 128 row blocks of 96 the
// call has too few workgroups to stream X at HBM speed, so K is cut into
// slices of at least 4 k-tiles until about 256 workgroups run.
int64_t lora_down_slices(int64_t m, int64_t k, int64_t rank) {
    const int64_t tiles = (m + TileLora96::BM - 1) / TileLora96::BM;
    const int64_t ktiles = (k * 2 + TileLora96::BK - 1) / TileLora96::BK;
    if (tiles >= 128 || rank > TileLora96::BN || rank % 4 || ktiles < 8) return 1;
    int64_t s = (256 + tiles - 1) / tiles;
    if (s > ktiles / 4) s = ktiles / 4;
    const int64_t per = (ktiles + s - 1) / s;
    return (ktiles + per - 1) / per;  // no empty slice
}

}  // namespace

int64_t lora_down_workspace_bytes(int64_t m, int64_t k, int64_t rank) {
    const int64_t s = lora_down_slices(m, k, rank);
    return s > 1 ? s * m * rank * 4 : 0;
}

hipError_t launch_lora_down(const GemmArgs& args, void* workspace, int64_t workspace_bytes, hipStream_t st) {
    const int64_t s = lora_down_slices(args.m, args.k, args.n);
    // The reduction stores 4 bf16 per lane: t rows 8-byte aligned.
    const bool t_vec = args.ldo % 4 == 0 && (uintptr_t)args.out % 8 == 0;
    if (s == 1 || !t_vec || workspace == nullptr || workspace_bytes < s * args.m * args.n * 4)
        return launch_gemm(kOpBF16, false, args, st);
    GemmArgs a = args;
    const int64_t ktiles = (a.k * 2 + TileLora96::BK - 1) / TileLora96::BK;
    a.kt_split = (ktiles + s - 1) / s;
    a.out = workspace;
    a.ldo = a.n;
    a.out_vec = 1;
    const int tiles_m = (int)((a.m + TileLora96::BM - 1) / TileLora96::BM);
    hipLaunchKernelGGL((gemm_kernel<TileLora96, kOpBF16, kEpiF32, false, true, false, false>),
                       dim3((unsigned)tiles_m, (unsigned)s), dim3(TileLora96::NT), 0, st, a, tiles_m, 1);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t threads = a.m * (a.n / 4);
    hipLaunchKernelGGL(lora_down_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       (const float*)workspace, (int)s, a.m, (int)a.n, (uint16_t*)args.out, args.ldo);
    return hipGetLastError();
}

hipError_t launch_gemm(int kind, bool raw_i32, const GemmArgs& args, hipStream_t st) {
    GemmArgs a = args;
    a.out_vec = (a.ldo % 4 == 0) && (a.n % 4 == 0) && ((uintptr_t)a.out % 16 == 0);
    const bool lora = a.lora_t != nullptr;
    if (kind != kOpBF16 && !raw_i32 && skinny_supported(a)) return launch_gemm_skinny(kind, a, st);
    if (kind != kOpBF16 && !raw_i32 && w4_supported(a)) return launch_gemm_w4(kind, a, st);
    if (kind == kOpE4M3)
        return lora ? launch_scaled<TileBigLora, kOpE4M3, true>(a, st) : launch_scaled<TileBig, kOpE4M3, false>(a, st);
    if (kind == kOpInt8) {
        if (raw_i32)
            return a.out_vec ? launch_tile<TileBig, kOpInt8, kEpiI32, false, true, false>(a, st)
                             : launch_tile<TileBig, kOpInt8, kEpiI32, false, false, false>(a, st);
        return lora ? launch_scaled<TileBigLora, kOpInt8, true>(a, st) : launch_scaled<TileBig, kOpInt8, false>(a, st);
    }
    if ((a.m + 95) / 96 <= 256)
        return a.out_vec ? launch_tile<TileLora96, kOpBF16, kEpiBF16, false, true, false>(a, st)
                         : launch_tile<TileLora96, kOpBF16, kEpiBF16, false, false, false>(a, st);
    return a.out_vec ? launch_tile<TileLora, kOpBF16, kEpiBF16, false, true, false>(a, st)
                     : launch_tile<TileLora, kOpBF16, kEpiBF16, false, false, false>(a, st);
}

}  // namespace h3q
