// Persistent scaled GEMM for large M on gfx950: four waves of 128 x 128.
//
//   out[m, n] = bf16( s_a[m] * (s_w[n] * float(sum_k A[m, k] * B[n, k])) [+ bias[n]] )
//
// A workgroup of four waves (one per SIMD) walks 256 x 256 output tiles
// blockIdx.x, blockIdx.x + gridDim.x, ... (one workgroup per CU).  Each wave
// owns a 128 x 128 block: 4 x 4 accumulators of the 32 x 32 MFMA
// (v_mfma_f32_32x32x64_f8f6f4 / v_mfma_i32_32x32x32_i8), 256 registers that
// live in the AGPR file for the whole kernel.  Per output element the MFMA
// pipe then needs half the LDS fragment reads of 64 x 64 wave blocks.
//
// K advances in 64-byte steps through a ring of four 32 KiB LDS stages
// (A 256 x 64 and B 256 x 64 codes each), filled by buffer_load_dwordx4 ...
// lds.  Step u (one per k-step, continuous across the tiles of a workgroup):
//   * 16 MFMAs (int8: 32) on the fragments of stage u, held in registers;
//   * the fragments of stage u + 1 read into the other register set;
//   * the 8 copy instructions of step u + 4 into stage u, which every wave
//     finished reading (into registers) before the barrier that ended step
//     u - 1;
//   * wait until the copies of step u + 2 have landed (vmcnt <= 16), barrier.
// A copy is thus issued two to three steps before it is read.
//
// Operand layouts in the stages:
//   * row-major (lda / ldb bytes per row): a row's 64 bytes are 4 chunks of
//     16, chunk c at c ^ swz(row), so the ds_read_b128 of 16 consecutive rows
//     at one chunk hit distinct banks;
//   * tiled (16-row x 128-byte blocks of 2 KiB in fragment order, see
//     include/taomate_h3_amd.h): a 64-byte step of a block is two 512-byte
//     pieces 1 KiB apart, copied as one 1 KiB wave instruction and read in
//     place (16 consecutive rows read 16 consecutive 16-byte slots).
//
// The per-row / per-column scale vectors and the bias of a tile are copied
// into LDS (double-buffered by tile parity) together with the tile's first
// k-step.  Their extra copy instruction makes some waits cover one more
// load than needed, never one less.
//
// Wait counts.  vmcnt counts loads and stores together.  Loads complete in
// issue order among themselves, so with two newer load groups (16 loads)
// outstanding behind the group a step needs, vmcnt <= 16 implies that group
// has landed whatever the pending epilogue stores do: stores only make the
// wait longer.
//
// Epilogue of a tile: the accumulators are read from the AGPRs, scaled in
// the reference order s_a * (s_w * acc) (fma with the bias), rounded to bf16,
// and staged per 32-row block through the ring stage whose contents the
// next step's fragments already hold in registers; each store then writes
// 4 rows x 256 contiguous bytes.  A barrier keeps copies out of that stage
// until every wave has read it back.
//
// The MFMAs are inline asm with their accumulator operand pinned to AGPRs
// ("a"); reading them back uses v_accvgpr_read after explicit wait states
// for the MFMA's passes.  Results are the bits of gemm_kernel / the
// persistent 16-wave kernel: the same instructions on the same operands in
// the same k order.
#include <stdint.h>

#include <type_traits>

#include "gemm_tiles.hpp"
#include "h3q_common.hpp"
#include "h3q_kernels.hpp"

namespace h3q {

namespace {

constexpr int kW4Stages = 4;
constexpr int kW4StageBytes = (256 + 256) * 64;  // 32 KiB
constexpr int kW4ABytes = 256 * 64;              // A part of a stage
// Outputs of at least this many bytes are stored with the non-temporal cache
// policy (gfx950 "nt"): they exceed what the caches could keep for a
// consumer anyway, and without the hint their dirty lines stay in the
// Infinity Cache and are written back under whatever runs next.  Measured at
// c2 (252 MB of output, act-quant then GEMM): step 516-518 -> 499-500 us,
// of which the following act-quant 37-38 -> 27-28 us and the GEMM 479 -> 472.
constexpr int64_t kW4StreamOutBytes = int64_t(64) << 20;
constexpr int kCachePolicyNT = 2;

// One wave copy (buffer_load_dwordx4 ... lds) with a scalar offset: lane L's
// 16 bytes at src + voff + soff land at LDS byte lds_base + 16 L.  Inline
// asm for the reason given at copy16 (h3q_common.hpp).
// The scalar operands go through readfirstlane: they are uniform, and where
// the compiler holds one in a VGPR (it may, in the LoRA instances) this moves
// it to an SGPR; on a value already in SGPRs it folds away.
__device__ __forceinline__ void copy16_soff(const CopySrc& src, uint32_t lds_base, uint32_t voff, uint32_t soff) {
    const v4i d = {__builtin_amdgcn_readfirstlane(src.d[0]), __builtin_amdgcn_readfirstlane(src.d[1]),
                   __builtin_amdgcn_readfirstlane(src.d[2]), __builtin_amdgcn_readfirstlane(src.d[3])};
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(d),
                   "s"(__builtin_amdgcn_readfirstlane(soff))
                 : "memory");
}

// MFMAs with the accumulator in AGPRs.  *_first starts a tile (srcC = 0).
__device__ __forceinline__ void mfma_e4m3(v16f& c, const v8i& b, const v8i& a) {
    asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a));
}
__device__ __forceinline__ void mfma_e4m3_first(v16f& c, const v8i& b, const v8i& a) {
    asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0" : "=a"(c) : "v"(b), "v"(a));
}
__device__ __forceinline__ void mfma_i8(v16i& c, const v4i& b, const v4i& a) {
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a));
}
__device__ __forceinline__ void mfma_i8_first(v16i& c, const v4i& b, const v4i& a) {
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0" : "=a"(c) : "v"(b), "v"(a));
}
// bf16 rank step of the LoRA epilogue: c (binary32 values in the
// accumulator registers, whatever acc_t says) += b x a.
template <class acc_t>
__device__ __forceinline__ void mfma_bf16(acc_t& c, const v4i& b, const v4i& a) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a));
}
// An accumulator register read as the binary32 value it holds (LORA: after
// the conversion every accumulator holds binary32, whatever acc_t says).
__device__ __forceinline__ float agpr_bits(float x) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(x));
    return v;
}
__device__ __forceinline__ float agpr_bits(int x) {
    int v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(x));
    return __int_as_float(v);
}
// Put 16 values computed in VGPRs into an accumulator's AGPRs.
template <class acc_t>
__device__ __forceinline__ void agpr_write(acc_t& c, const acc_t& v) {
    asm volatile("; accumulator <- vgprs" : "=a"(c) : "0"(v));
}
__device__ __forceinline__ float agpr_read(float x) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(x));
    return v;
}
__device__ __forceinline__ float agpr_read(int x) {
    int v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(x));
    return (float)v;
}

// Chunk swizzle of a 64-byte row-major stage row (conflict-free ds_read_b128
// of 16 consecutive rows at one logical chunk).
__device__ __forceinline__ int swz64(int r) { return (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2); }

template <int OP>
struct W4Op;
template <>
struct W4Op<kOpE4M3> {
    using acc_t = v16f;
    using frag_t = v8i;
    static constexpr int kSteps = 1;  // MFMA k-steps per 64-byte stage
};
template <>
struct W4Op<kOpInt8> {
    using acc_t = v16i;
    using frag_t = v4i;
    static constexpr int kSteps = 2;
};

}  // namespace

// F16: binary16 output and bias instead of bf16 (a separate instance, so the
// bf16 epilogue carries no select).  stream_out: the output stores carry the
// non-temporal cache policy.
//
// Schedule.  Workgroup b takes tiles b, b + G, ... (G = gridDim.x).  When the
// last round of tiles is at most half full (0 < T % G <= G / 2 for T tiles)
// and split_tail is set, that round's tiles are cut into two 128 x 256 halves
// instead, and every workgroup b < 2 (T % G) finishes with one half (tile
// rounds * G + b % (T % G), rows 128 * (b / (T % G)) ..): the last round then
// keeps every CU busy for about half a round instead of leaving half the CUs
// idle for a full one.  A half tile runs the same ring and k order with two
// 32-row blocks per wave (waves 2 x 2 of 64 x 128), so its outputs carry the
// same bits as in a whole tile.
//
// LORA: out gains lora_scale * (t[m, :] . lora_b[n, :]) (bf16 t [M, r] and
// lora_b [N, r], r <= 128) before the single rounding.  Each tile's copy
// stream carries four more groups after its k-steps: rank bytes
// 64 l .. 64 l + 63 of t (as A) and of lora_b (as B), row-major, zero past
// 2 r bytes.  After the last k-step every accumulator becomes
// y = s_a * (s_w * acc) [+ bias] times RN(1 / lora_scale) (exactly y when
// the scale is 1); then four rank steps run through the ring like k-steps,
// each v_mfma_f32_32x32x16_bf16 adding t . lora_b to y in rank order, and the
// epilogue stores bf16(lora_scale * acc) (acc itself when the scale is 1).
// The ring never drains: the rank steps' copy slots already carry the next
// tile's first groups.
template <int OP, bool BIAS, bool TA, bool TB, bool F16, bool LORA>
__global__ __launch_bounds__(256, 1) void gemm_w4_kernel(GemmArgs p, int tiles_m, int tiles_n, int split_tail,
                                                        int stream_out) {
    using acc_t = typename W4Op<OP>::acc_t;
    using frag_t = typename W4Op<OP>::frag_t;
    constexpr int KS = W4Op<OP>::kSteps;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_ring[kW4Stages * kW4StageBytes];
    // Per tile parity: row scales [256] f32 | column scales [256] f32 | bias [256] bf16.
    __shared__ __attribute__((aligned(1024))) uint8_t lds_ep[2 * 3 * 1024];
    H3Q_LDS uint8_t* const ring = (H3Q_LDS uint8_t*)lds_ring;
    H3Q_LDS uint8_t* const ep = (H3Q_LDS uint8_t*)lds_ep;
    const uint32_t ring_addr = (uint32_t)(uintptr_t)ring;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wn0 = (wave & 1) * 128;
    const int g = lane >> 5, c32 = lane & 31;
    const int ksteps = (int)(p.k / 64);          // even: k % 128 == 0
    const int ngroups = ksteps + (LORA ? 4 : 0); // copy groups per tile
    const int64_t steps128 = p.k / 128;          // tiled operands: 128-byte k-steps per block row

    // Work items j < nfull are whole tiles; item nfull (has_half) is a half tile.
    const int T = tiles_m * tiles_n, G = (int)gridDim.x, b = (int)blockIdx.x;
    const int rounds = T / G, rem = T % G;
    const bool split = split_tail != 0 && rem > 0 && 2 * rem <= G;
    const int nfull = split ? rounds : (T - b + G - 1) / G;
    int half_tm = 0, half_tn = 0, half_m0 = 0;
    bool has_half = false;
    if (split && b < 2 * rem) {
        tile_coords(rounds * G + b % rem, tiles_m, tiles_n, half_tm, half_tn);
        half_m0 = half_tm * 256 + 128 * (b / rem);
        has_half = p.m > half_m0;
    }
    const int ntiles = nfull + (has_half ? 1 : 0);
    if (ntiles == 0) return;

    const bool row_scales = p.a_scale_per_row != 0, col_scales = p.b_scale_per_col != 0;
    // A per-tensor scale fills its vector (both parities) once.
    if (!row_scales || !col_scales) {
        const float sa0 = row_scales ? 0.0f : p.a_scale[0], sw0 = col_scales ? 0.0f : p.b_scale[0];
        for (int c = threadIdx.x; c < 2 * 256; c += 256) {
            H3Q_LDS float* e = (H3Q_LDS float*)(ep + (c >> 8) * 3072);
            if (!row_scales) e[c & 255] = sa0;
            if (!col_scales) e[256 + (c & 255)] = sw0;
        }
    }

    // Every lambda below is force-inlined: an outlined one would take its
    // captures through private memory, and the copy instructions' scalar
    // operands (descriptors, LDS bases, offsets) would stop being uniform.
    struct TileSrc {
        int m0, n0, rows, cols;
    };
    auto tile_src = [&](int j) __attribute__((always_inline)) {
        TileSrc t;
        int tm, tn;
        if (j < nfull) {
            tile_coords(b + j * G, tiles_m, tiles_n, tm, tn);
            t.m0 = tm * 256;
        } else {
            tn = half_tn;
            t.m0 = half_m0;
        }
        const int mrows = j < nfull ? 256 : 128;
        t.n0 = tn * 256;
        t.rows = (int)(p.m - t.m0 < mrows ? p.m - t.m0 : mrows);
        t.cols = (int)(p.n - t.n0 < 256 ? p.n - t.n0 : 256);
        return t;
    };

    // ---------------------------------------------------------------- copies
    // Descriptors and per-lane offsets of the tile being fetched; the k-step
    // enters as the scalar offset.  Past the last tile the descriptors are
    // empty, so the trailing copies read zeros into stages nobody reads.  A
    // half tile's A rows past 128 are out of range too (zeros, never read).
    CopySrc ra(nullptr, 0), rb(nullptr, 0);
    uint32_t voff_a[4], voff_b[4];
    // LORA: rows / columns of the copy tile, kept as scalars for the rank
    // groups' descriptors and offsets (tile_src costs several integer
    // divisions).
    int cp_m0 = 0, cp_n0 = 0, cp_rows = 0, cp_cols = 0;
    int rank_chunk16 = 0;  // LORA: byte of the lane's 16-byte chunk inside a rank group
    int cj = 0, cs = 0;  // tile / k-step of the next copy group
    auto operand_offset = [&](bool tiled, int c, int sub_row, int pos, int ln, int rows, int64_t ld) __attribute__((always_inline)) -> uint32_t {
        if (tiled) {  // 16-row block c
            const int nblk = (rows + 15) / 16;
            return c < nblk ? (uint32_t)(c * steps128 * 2048) + (uint32_t)((ln >> 5) * 1024 + (ln & 31) * 16)
                            : 0x80000000u;
        }
        const int row = c * 16 + sub_row;  // 16 rows x 64 bytes per copy
        return row < rows ? (uint32_t)row * (uint32_t)ld + (uint32_t)((pos ^ swz64(sub_row)) * 16) : 0x80000000u;
    };
    auto setup_copy_tile = [&](int j) __attribute__((always_inline)) {
        const bool live = j < ntiles;
        const TileSrc t = tile_src(live ? j : ntiles - 1);
        const uint32_t a_bytes = TA ? (uint32_t)((t.rows + 15) / 16 * steps128 * 2048) : (uint32_t)((int64_t)t.rows * p.lda);
        const uint32_t b_bytes = TB ? (uint32_t)((t.cols + 15) / 16 * steps128 * 2048) : (uint32_t)((int64_t)t.cols * p.ldb);
        ra = CopySrc((const uint8_t*)p.a + (TA ? (int64_t)(t.m0 / 16) * steps128 * 2048 : (int64_t)t.m0 * p.lda),
                     live ? a_bytes : 0u);
        rb = CopySrc((const uint8_t*)p.b + (TB ? (int64_t)(t.n0 / 16) * steps128 * 2048 : (int64_t)t.n0 * p.ldb),
                     live ? b_bytes : 0u);

        if constexpr (LORA) {
            cp_m0 = t.m0;
            cp_n0 = t.n0;
            cp_rows = live ? t.rows : 0;  // no rows: the rank copies past the last tile read zeros
            cp_cols = live ? t.cols : 0;
        }
        const int ln = opaque_lane();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = wave + 4 * i;
            voff_a[i] = operand_offset(TA, c, ln >> 2, ln & 3, ln, t.rows, p.lda);
            voff_b[i] = operand_offset(TB, c, ln >> 2, ln & 3, ln, t.cols, p.ldb);
        }
    };
    // Epilogue vectors of tile j into LDS (waves 0, 1, 2: one copy each).
    auto issue_vectors = [&](int j) __attribute__((always_inline)) {
        if (j >= ntiles) return;
        const TileSrc t = tile_src(j);
        H3Q_LDS uint8_t* e = ep + (j & 1) * 3072;
        if (wave == 0 && row_scales)
            copy16(CopySrc(p.a_scale + t.m0, (uint32_t)t.rows * 4u), (uint32_t)(uintptr_t)e, 16u * lane);
        if (wave == 1 && col_scales)
            copy16(CopySrc(p.b_scale + t.n0, (uint32_t)t.cols * 4u), (uint32_t)(uintptr_t)(e + 1024), 16u * lane);
        if (BIAS && wave == 2)
            copy16(CopySrc(p.bias + t.n0, (uint32_t)t.cols * 2u), (uint32_t)(uintptr_t)(e + 2048),
                   lane < 32 ? 16u * lane : 0x80000000u);
    };
    // LORA rank groups of the copy tile: once its k-step groups are all
    // issued, ra / rb and voff_a / voff_b (free until the next tile's set-up)
    // take the rows of t and lora_b, 16 rows x 64 bytes per copy, row-major;
    // group l adds 64 l bytes as the scalar offset.
    auto setup_rank_copies = [&]() __attribute__((always_inline)) {
        ra = CopySrc((const uint8_t*)p.lora_t + (int64_t)cp_m0 * p.ldt * 2, (uint32_t)(cp_rows * p.ldt * 2));
        rb = CopySrc((const uint8_t*)p.lora_b + (int64_t)cp_n0 * p.ldlb * 2, (uint32_t)(cp_cols * p.ldlb * 2));
        const int ln = opaque_lane();
        rank_chunk16 = 16 * ((ln & 3) ^ swz64(ln >> 2));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = (wave + 4 * i) * 16 + (ln >> 2);
            voff_a[i] = row < cp_rows ? (uint32_t)row * (uint32_t)(p.ldt * 2) + (uint32_t)rank_chunk16 : 0x80000000u;
            voff_b[i] = row < cp_cols ? (uint32_t)row * (uint32_t)(p.ldlb * 2) + (uint32_t)rank_chunk16 : 0x80000000u;
        }
    };
    // Copy q (0..3: A, 4..7: B) of the group for (cj, cs) into stage st.
    // rank: the group is a LORA rank group (the tile's last four steps issue
    // those; a compile-time flag keeps the branch out of the other steps).
    auto issue_copy = [&](int q, int st, auto rank) __attribute__((always_inline)) {
        const uint32_t base = ring_addr + (uint32_t)(st * kW4StageBytes);
        if constexpr (decltype(rank)::value) {
            // Rank bytes 64 l + 16 chunk .. + 15 of the lane's row; zero past
            // 2 r (a lane whose chunk starts there gets an out-of-range offset).
            const int l = cs - ksteps;
            const bool in = rank_chunk16 < 2 * (int)p.lora_rank - 64 * l;
            if (q < 4)
                copy16_soff(ra, base + (uint32_t)((wave + 4 * q) * 1024), in ? voff_a[q] : 0x80000000u,
                            (uint32_t)(64 * l));
            else
                copy16_soff(rb, base + (uint32_t)(kW4ABytes + (wave + 4 * (q - 4)) * 1024),
                            in ? voff_b[q - 4] : 0x80000000u, (uint32_t)(64 * l));
            return;
        }
        const uint32_t soff_t = (uint32_t)((cs >> 1) * 2048 + (cs & 1) * 512), soff_r = (uint32_t)(cs * 64);
        if (q < 4)
            copy16_soff(ra, base + (uint32_t)((wave + 4 * q) * 1024), voff_a[q], TA ? soff_t : soff_r);
        else
            copy16_soff(rb, base + (uint32_t)(kW4ABytes + (wave + 4 * (q - 4)) * 1024), voff_b[q - 4],
                        TB ? soff_t : soff_r);
    };
    auto advance_copy = [&]() __attribute__((always_inline)) {
        if (++cs == ngroups) {
            cs = 0;
            ++cj;
            setup_copy_tile(cj);
            issue_vectors(cj);
        }
    };

    // ------------------------------------------------------ fragment reads
    // Stage-relative byte offsets of this lane's fragment halves: rows
    // wm0 + c32 (A) and wn0 + c32 (B) of the first 32-row block; block i adds
    // 2048 in either layout.  e4m3: halves h = 0, 1 of the 32-byte fragment
    // (k bytes 32 g + 16 h); int8: k-steps s = 0, 1 (k bytes 32 s + 16 g).
    // A whole tile puts a wave's rows at wm0 = 128 (wave / 2), a half tile at
    // 64 (wave / 2); rda holds the offsets of the layout being read.
    uint32_t rda[2], rda_half[2], rdb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int chunk = OP == kOpE4M3 ? 2 * g + h : 2 * h + g;      // logical 16-byte chunk of the row
        const int tiled_off = ((c32 & 15) + 16 * (OP == kOpE4M3 ? g : h)) * 16 + (OP == kOpE4M3 ? h : g) * 512;
        auto a_off = [&](int wm0) __attribute__((always_inline)) {
            return TA ? (uint32_t)(((wm0 + c32) >> 4) * 1024 + tiled_off)
                      : (uint32_t)((wm0 + c32) * 64 + ((chunk ^ swz64(c32)) << 4));
        };
        rda[h] = a_off((wave >> 1) * 128);
        rda_half[h] = a_off((wave >> 1) * 64);
        rdb[h] = kW4ABytes + (TB ? (uint32_t)(((wn0 + c32) >> 4) * 1024 + tiled_off)
                                 : (uint32_t)((wn0 + c32) * 64 + ((chunk ^ swz64(c32)) << 4)));
    }
    // Rank groups (LORA) sit row-major in the stage: rank k-step s of a
    // 64-byte row is logical chunk 2 s + g, as for the int8 fragments.
    uint32_t rra[2], rra_half[2], rrb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t chunk = (uint32_t)(((2 * h + g) ^ swz64(c32)) << 4);
        rra[h] = (uint32_t)(((wave >> 1) * 128 + c32) * 64) + chunk;
        rra_half[h] = (uint32_t)(((wave >> 1) * 64 + c32) * 64) + chunk;
        rrb[h] = (uint32_t)(kW4ABytes + (wn0 + c32) * 64) + chunk;
    }
    auto to_half_layout = [&]() __attribute__((always_inline)) {
        rda[0] = rda_half[0];
        rda[1] = rda_half[1];
        rra[0] = rra_half[0];
        rra[1] = rra_half[1];
    };
    struct Frags {
        frag_t a[4 * KS], b[4 * KS];
    };
    auto ld16 = [&](const H3Q_LDS uint8_t* ptr) __attribute__((always_inline)) -> v4i { return *(const H3Q_LDS v4i*)ptr; };
    // Fragment x of stage st for MI 32-row A blocks per wave: x < MI * KS
    // reads A block x % MI (k-step x / MI), the rest B block (x - MI KS) % 4
    // (k-step (x - MI KS) / 4).
    auto read_frag = [&](auto mi, Frags& F, int x, int st) __attribute__((always_inline)) {
        constexpr int MI = decltype(mi)::value;
        const H3Q_LDS uint8_t* sb = ring + st * kW4StageBytes;
        const bool is_a = x < MI * KS;
        const int xx = is_a ? x : x - MI * KS;
        const int y = is_a ? xx % MI : xx % 4, s = is_a ? xx / MI : xx / 4;
        if constexpr (OP == kOpE4M3) {
            const uint32_t* off = is_a ? rda : rdb;
            const v8i f = __builtin_shufflevector(ld16(sb + off[0] + y * 2048), ld16(sb + off[1] + y * 2048), 0, 1, 2,
                                                  3, 4, 5, 6, 7);
            if (is_a) F.a[y] = f;
            else F.b[y] = f;
        } else {
            const v4i f = ld16(sb + (is_a ? rda[s] : rdb[s]) + y * 2048);
            if (is_a) F.a[y + 4 * s] = f;
            else F.b[y + 4 * s] = f;
        }
    };

    // Rank fragment x (0..15) of stage st: x < 8 is t block x % 4, rank k-step
    // x / 4; the rest lora_b block x % 4, k-step (x - 8) / 4.  Held in the
    // fragment registers: e4m3 puts k-step s in lanes 4 s .. 4 s + 3 of the
    // block's v8i, int8 in element y + 4 s.
    auto read_rank = [&](Frags& F, int x, int st) __attribute__((always_inline)) {
        const H3Q_LDS uint8_t* sb = ring + st * kW4StageBytes;
        const bool is_a = x < 8;
        const int y = x & 3, s = (x & 7) >> 2;
        const v4i f = ld16(sb + (is_a ? rra[s] : rrb[s]) + y * 2048);
        frag_t* dst = is_a ? F.a : F.b;
        if constexpr (OP == kOpE4M3) {
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[y][4 * s + e] = f[e];
        } else {
            dst[y + 4 * s] = f;
        }
    };
    auto rank_frag = [&](const frag_t* f, int y, int s) __attribute__((always_inline)) -> v4i {
        if constexpr (OP == kOpE4M3) {
            return s == 0 ? __builtin_shufflevector(f[y], f[y], 0, 1, 2, 3)
                          : __builtin_shufflevector(f[y], f[y], 4, 5, 6, 7);
        } else {
            return f[y + 4 * s];
        }
    };

    acc_t acc[4][4];
    Frags F0, F1;
    // MFMA t of a step: acc[i][j] += b-fragment j x a-fragment i (k-step s).
    auto mfma = [&](auto mi, bool first, const Frags& Fc, int t) __attribute__((always_inline)) {
        constexpr int MI = decltype(mi)::value;
        const int s = t / (4 * MI), i = (t % (4 * MI)) / 4, j = t % 4;
        if constexpr (OP == kOpE4M3) {
            if (first) mfma_e4m3_first(acc[i][j], Fc.b[j], Fc.a[i]);
            else mfma_e4m3(acc[i][j], Fc.b[j], Fc.a[i]);
        } else {
            if (first && s == 0) mfma_i8_first(acc[i][j], Fc.b[j + 4 * s], Fc.a[i + 4 * s]);
            else mfma_i8(acc[i][j], Fc.b[j + 4 * s], Fc.a[i + 4 * s]);
        }
    };
    // One step's instruction stream: every MFMA is followed by the next
    // fragment read (first NR slots) and, in every CP-th slot, a copy, each
    // slot kept in place by a scheduling barrier.  The reads of the next stage use the
    // layout of MI = 4 (a superset of a half tile's: the extra A blocks are
    // read and never used), so a step may prepare a half tile's first step.
    // LORA, after the last k-step of a tile: accumulator block (i, j) becomes
    // y = s_a * (s_w * acc) [+ bias] (the epilogue's arithmetic), times
    // RN(1 / lora_scale), as binary32 in the accumulator registers; the rank
    // steps then add t . lora_b to it.  conv_e points at the tile's epilogue
    // vectors.
    const H3Q_LDS uint8_t* conv_e = ep;
    // The blocks go column block by column block (j outer), so each lane
    // reads the column scales and bias of a column block once (cw, cb) and
    // its MI row scales once (ca).
    float ca[4];
    v4f cw[4];
    v2u cb[4];
    auto conv_row_scales = [&](auto mi) __attribute__((always_inline)) {
        constexpr int MI = decltype(mi)::value;
        const int wm0 = (wave >> 1) * 32 * MI;
#pragma unroll
        for (int i = 0; i < MI; ++i) ca[i] = ((const H3Q_LDS float*)conv_e)[wm0 + 32 * i + (lane & 31)];
    };
    auto conv_col_vectors = [&](int j) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int col = wn0 + 32 * j + 8 * q + 4 * (lane >> 5);
            cw[q] = *(const H3Q_LDS v4f*)(conv_e + 1024 + 4 * col);
            if constexpr (BIAS) cb[q] = *(const H3Q_LDS v2u*)(conv_e + 2048 + 2 * col);
        }
    };
    auto convert_block = [&](int i, int j) __attribute__((always_inline)) {
        // RN(1 / lora_scale) is 1 for a unit scale, and v * 1 = v exactly, so
        // the multiply runs unconditionally (a select would cost as much).
        const float rs = 1.0f / p.lora_scale;
        const float sa = ca[i];
        acc_t y;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const v4f sw4 = cw[q];
            const v2u b4 = cb[q];
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const float t = __fmul_rn(sw4[x], agpr_read(acc[i][j][4 * q + x]));
                float v;
                if constexpr (BIAS) v = __builtin_fmaf(sa, t, (x & 1) ? bf16_hi(b4[x >> 1]) : bf16_lo(b4[x >> 1]));
                else v = __fmul_rn(sa, t);
                v = __fmul_rn(v, rs);
                if constexpr (OP == kOpE4M3) y[4 * q + x] = v;
                else y[4 * q + x] = __float_as_int(v);
            }
        }
        agpr_write(acc[i][j], y);
    };
    // kind: 0 a k-step (MFMAs of the codes), 1 a LORA rank step (bf16 MFMAs),
    // 2 the first rank step, which converts block b = (b % MI, b / MI) in slot
    // b and runs block b's first MFMA one slot later (the conversions' VALU
    // work overlaps the MFMAs, and no MFMA reads an accumulator right after
    // its VALU write);
    // next: the fragments read for the next step are 0 codes, 1 rank.
    auto body = [&](auto mi, auto rank, auto kind, auto next, bool first, const Frags& Fc, Frags& Fn, int rst,
                    int cst) __attribute__((always_inline)) {
        constexpr int MI = decltype(mi)::value;
        constexpr int KIND = decltype(kind)::value;
        constexpr bool RANK = KIND != 0, CONV = KIND == 2, NEXT_RANK = decltype(next)::value != 0;
        constexpr int NM = RANK ? 8 * MI : 4 * MI * KS;          // MFMAs per step per wave
        constexpr int NR = NEXT_RANK ? 16 : (4 + 4) * KS;        // fragment reads per step
        constexpr int NMS = CONV ? NM + 1 : NM;                  // MFMA slots (the first one converts only)
        constexpr int NT = NMS > NR + 8 ? NMS : NR + 8;
        // The 8 copies go to every CP-th slot over the whole step rather than
        // 8 consecutive slots after the reads: the four waves' copies then
        // reach the texture unit spread over the step (e4m3 c2 step 0.8%
        // faster) and, in steps of half-length MFMAs (int8, rank steps), each
        // copy's scalar set-up sits under more than one MFMA.
        constexpr int CP = NT / 8;
        if constexpr (CONV) {
            conv_row_scales(mi);
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if constexpr (CONV) {
                if (t < 4 * MI) {
                    if (t % MI == 0) conv_col_vectors(t / MI);
                    convert_block(t % MI, t / MI);
                }
                __builtin_amdgcn_sched_barrier(0);  // the MFMA below reads the block converted one slot earlier
            }
            const int tm = CONV ? t - 1 : t;  // MFMA of this slot
            if (tm >= 0 && tm < NM) {
                if constexpr (RANK) {
                    const int s = tm / (4 * MI);
                    // the converting step takes its first 4 MI MFMAs in conversion order
                    const int i = CONV && s == 0 ? tm % MI : (tm % (4 * MI)) / 4;
                    const int j = CONV && s == 0 ? tm / MI : tm % 4;
                    mfma_bf16(acc[i][j], rank_frag(Fc.b, j, s), rank_frag(Fc.a, i, s));
                } else {
                    mfma(mi, first, Fc, tm);
                }
            }
            if (t < NR) {
                if constexpr (NEXT_RANK) read_rank(Fn, t, rst);
                else read_frag(std::integral_constant<int, 4>(), Fn, t, rst);
            }
            if (t % CP == CP - 1 && t / CP < 8) issue_copy(t / CP, cst, rank);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ------------------------------------------------------------- epilogue
    auto epilogue = [&](auto mi, int mj, int st) __attribute__((always_inline)) {
        constexpr int MI = decltype(mi)::value;
        const int wm0 = (wave >> 1) * 32 * MI;
        const TileSrc cur = tile_src(mj);
        const int ln = opaque_lane();
        const int gg = ln >> 5, cc = ln & 31;
        const H3Q_LDS uint8_t* e = ep + (mj & 1) * 3072;
        H3Q_LDS uint8_t* const scratch = ring + st * kW4StageBytes + wave * 8192;
        const __amdgpu_buffer_rsrc_t ro =
            make_rsrc((uint8_t*)p.out + (int64_t)cur.m0 * p.ldo * 2, (uint32_t)((int64_t)cur.rows * p.ldo * 2));
        // This lane's vectors, read once (before any scratch write): row
        // scales of rows wm0 + 32 i + cc; column scales and bias of columns
        // wn0 + 8 g16 + 4 gg + x, g16 = 4 jj + q.
        float sa[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) sa[i] = ((const H3Q_LDS float*)e)[wm0 + 32 * i + cc];
        v4f sw4[16];
        v2u b4[16];
#pragma unroll
        for (int g16 = 0; g16 < 16; ++g16) {
            const int nl = wn0 + 8 * g16 + 4 * gg;
            sw4[g16] = *(const H3Q_LDS v4f*)(e + 1024 + 4 * nl);
            if constexpr (BIAS) b4[g16] = *(const H3Q_LDS v2u*)(e + 2048 + 2 * nl);
        }
        // Store columns of this lane: 8 bf16 at wn0 + 8 (ln % 16).
        const int col8 = wn0 + 8 * (ln & 15);
        const bool col_ok = col8 < cur.cols;
        // VALU reads of MFMA results: wait out the last MFMAs' passes.
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
            for (int g16 = 0; g16 < 16; ++g16) {
                const int jj = g16 >> 2, q = g16 & 3;
                float y[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    if constexpr (LORA) {  // y + t . lora_b, scaled back
                        const float v = agpr_bits(acc[i][jj][4 * q + x]);
                        y[x] = __fmul_rn(p.lora_scale, v);  // exact for a unit scale
                        continue;
                    }
                    const float t = __fmul_rn(sw4[g16][x], agpr_read(acc[i][jj][4 * q + x]));
                    if constexpr (BIAS) {
                        const uint32_t w = b4[g16][x >> 1];
                        y[x] = __builtin_fmaf(sa[i], t, (x & 1) ? out_hi(w, F16) : out_lo(w, F16));
                    } else {
                        y[x] = __fmul_rn(sa[i], t);
                    }
                }
                // row cc of the block, columns 8 g16 + 4 gg .. + 3 of the wave
                *(H3Q_LDS v2u*)(scratch + cc * 256 + ((g16 ^ (cc & 15)) << 4) + gg * 8) =
                    v2u{pack_out2(y[0], y[1], F16), pack_out2(y[2], y[3], F16)};
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int row = 4 * r + (ln >> 4);
                const v4u v = *(const H3Q_LDS v4u*)(scratch + row * 256 + (((ln & 15) ^ (row & 15)) << 4));
                const uint32_t off =
                    col_ok ? ((uint32_t)(wm0 + 32 * i + row) * (uint32_t)p.ldo + (uint32_t)(cur.n0 + col8)) * 2u
                           : 0xFFFFFFF0u;
                if (stream_out) __builtin_amdgcn_raw_buffer_store_b128(v, ro, off, 0, kCachePolicyNT);
                else __builtin_amdgcn_raw_buffer_store_b128(v, ro, off, 0, 0);
            }
        }
    };

    // ------------------------------------------------------------ main loop
    // Prime the ring: the copy cursor's next four groups into stages 0..3,
    // then the fragments of stage 0.
    auto prime = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < kW4Stages; ++st) {
#pragma unroll
            for (int q = 0; q < 8; ++q) issue_copy(q, st, std::false_type());
            advance_copy();
        }
        wait_vmcnt<(kW4Stages - 1) * 8>();
        ring_barrier();
#pragma unroll
        for (int x = 0; x < 8 * KS; ++x) read_frag(std::integral_constant<int, 4>(), F0, x, 0);
        wait_vmcnt<(kW4Stages - 2) * 8>();
        ring_barrier();
    };
    setup_copy_tile(0);
    issue_vectors(0);
    if (nfull == 0) to_half_layout();
    prime();

    int cur_st = 0;  // stage of the running step (its fragments are in registers)
    const std::integral_constant<int, 0> codes_k;
    const std::integral_constant<int, 1> rank_k;
    const std::integral_constant<int, 2> conv_k;
    auto step = [&](auto mi, bool first, const Frags& Fc, Frags& Fn, auto rank, auto kind, auto next)
                    __attribute__((always_inline)) {
        const int nxt_st = cur_st + 1 == kW4Stages ? 0 : cur_st + 1;
        body(mi, rank, kind, next, first, Fc, Fn, nxt_st, cur_st);
        advance_copy();
        wait_vmcnt<(kW4Stages - 2) * 8>();
        ring_barrier();
        cur_st = nxt_st;
    };
    // One tile: ksteps steps (the last one reads the next tile's first
    // fragments, in the half layout when a half tile follows), then the
    // epilogue through the stage that is free until the next step's copies.
    // LORA: the last steps copy the rank groups instead; after the fold and
    // the epilogue the ring is primed again from stage 0.
    auto run_tile = [&](auto mi, int mj, bool next_half) __attribute__((always_inline)) {
        const std::integral_constant<int, decltype(mi)::value> m;
        const std::false_type op;
        if constexpr (!LORA) {
            step(m, true, F0, F1, op, codes_k, codes_k);
            if (ksteps == 2 && next_half) to_half_layout();
            step(m, false, F1, F0, op, codes_k, codes_k);
            for (int s = 2; s < ksteps; s += 2) {
                step(m, false, F0, F1, op, codes_k, codes_k);
                if (s + 2 == ksteps && next_half) to_half_layout();
                step(m, false, F1, F0, op, codes_k, codes_k);
            }
        } else {
            // Step s copies group s + 4: the rank groups in steps ksteps - 4 ..
            // ksteps - 1 (ksteps is even and at least 4), the next tile's first
            // groups in the four rank steps.  The last k-step reads the first
            // rank fragments; the last rank step the next tile's first ones.
            // The copy cursor runs four groups ahead: it reaches the rank
            // groups (cs == ksteps) as step ksteps - 4 begins.
            const std::true_type rk;
            if (ksteps > 4) {
                step(m, true, F0, F1, op, codes_k, codes_k);
                step(m, false, F1, F0, op, codes_k, codes_k);
                for (int s = 2; s < ksteps - 4; s += 2) {
                    step(m, false, F0, F1, op, codes_k, codes_k);
                    step(m, false, F1, F0, op, codes_k, codes_k);
                }
                setup_rank_copies();
                step(m, false, F0, F1, rk, codes_k, codes_k);
            } else {
                setup_rank_copies();
                step(m, true, F0, F1, rk, codes_k, codes_k);
            }
            step(m, false, F1, F0, rk, codes_k, codes_k);
            step(m, false, F0, F1, rk, codes_k, codes_k);
            step(m, false, F1, F0, rk, codes_k, rank_k);
            conv_e = ep + (mj & 1) * 3072;
            step(m, false, F0, F1, op, conv_k, rank_k);
            step(m, false, F1, F0, op, rank_k, rank_k);
            step(m, false, F0, F1, op, rank_k, rank_k);
            if (next_half) to_half_layout();
            step(m, false, F1, F0, op, rank_k, codes_k);
        }
        epilogue(m, mj, cur_st);
        ring_barrier();
    };
    for (int mj = 0; mj < nfull; ++mj) run_tile(std::integral_constant<int, 4>(), mj, has_half && mj + 1 == nfull);
    if (has_half) run_tile(std::integral_constant<int, 2>(), nfull, false);
    wait_vmcnt<0>();
}

bool w4_supported(const GemmArgs& a) {
    // k in 128-byte steps (at least two, so each tile spans four ring stages),
    // 8-column bf16 stores, a 16-byte aligned output, and the 32-bit
    // block-relative offsets of the copies and stores.
    if (a.k % 128 || a.k < 256 || a.n % 8 || a.ldo % 8 || (uintptr_t)a.out % 16) return false;
    if (a.out_f16 && a.a_tiled) return false;  // binary16 output: row-major activations only
    // LoRA: bf16 output, rank <= 128 in steps of 8 (checked by the C ABI).
    if (a.lora_t && (a.out_f16 || a.lora_rank > 128)) return false;
    if (a.m <= kSkinnyMaxM) return false;
    const int64_t tiled_block_row = (a.k / 128) * 2048 * 16;  // 256 rows of a tiled operand
    if ((a.a_tiled && tiled_block_row >= (int64_t(1) << 31)) || (a.b_tiled && tiled_block_row >= (int64_t(1) << 31)))
        return false;
    return 256 * a.ldo * 2 < (int64_t(1) << 31);
}

template <int OP, bool BIAS>
static hipError_t launch_w4_op(const GemmArgs& a, hipStream_t st) {
    const int tiles_m = (int)((a.m + 255) / 256), tiles_n = (int)((a.n + 255) / 256);
    const dim3 grid((unsigned)persistent_grid(tiles_m * tiles_n));
    const int stream_out = a.m * a.ldo * 2 >= kW4StreamOutBytes;
#define H3Q_W4(TA, TB, F16, LORA) \
    hipLaunchKernelGGL((gemm_w4_kernel<OP, BIAS, TA, TB, F16, LORA>), grid, dim3(256), 0, st, a, tiles_m, tiles_n, 1, \
                       stream_out)
    if (a.lora_t) {
        if (a.a_tiled) {
            if (a.b_tiled) H3Q_W4(true, true, false, true);
            else H3Q_W4(true, false, false, true);
        } else {
            if (a.b_tiled) H3Q_W4(false, true, false, true);
            else H3Q_W4(false, false, false, true);
        }
    } else if (a.out_f16) {
        if (a.b_tiled) H3Q_W4(false, true, true, false);
        else H3Q_W4(false, false, true, false);
    } else if (a.a_tiled) {
        if (a.b_tiled) H3Q_W4(true, true, false, false);
        else H3Q_W4(true, false, false, false);
    } else {
        if (a.b_tiled) H3Q_W4(false, true, false, false);
        else H3Q_W4(false, false, false, false);
    }
#undef H3Q_W4
    return hipGetLastError();
}

hipError_t launch_gemm_w4(int kind, const GemmArgs& a, hipStream_t st) {
    if (kind == kOpE4M3) return a.bias ? launch_w4_op<kOpE4M3, true>(a, st) : launch_w4_op<kOpE4M3, false>(a, st);
    return a.bias ? launch_w4_op<kOpInt8, true>(a, st) : launch_w4_op<kOpInt8, false>(a, st);
}

}  // namespace h3q
