// Shared device helpers for the gfx950 (CDNA4) quantized-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "quant_math.h"

namespace h3q {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

#define H3Q_LDS __attribute__((address_space(3)))

// Code formats (mirrored by include/taomate_h3_amd.h).
enum Format : int { kFmtE4M3 = 0, kFmtInt8 = 1 };
// Rounding forms of a per-row quantizer.
enum Rounding : int { kRoundDiv = 0, kRoundRcpMul = 1 };

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// binary32 -> bf16 bits, round to nearest even (finite inputs; NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t b = __float_as_uint(f);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (b >> 16) | 0x40u;
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// Two binary32 values -> two bf16 (round to nearest even) in one word, low
// half first: gfx950's v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{lo, hi}, v2bf));
}

// Two binary32 values -> two IEEE binary16 (round to nearest even, overflow
// to infinity) in one word, low half first.  The values are pinned as
// binary32 first: otherwise the compiler may fold a preceding fmaf into a
// mixed-precision FMA that rounds the exact result to binary16 once, where
// the epilogue rounds to binary32 and then to binary16.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    asm volatile("" : "+v"(lo), "+v"(hi));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}
__device__ __forceinline__ float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

// Output elements of the scaled GEMMs (and their bias): bf16, or binary16
// when f16 (a uniform kernel argument).
__device__ __forceinline__ uint32_t pack_out2(float lo, float hi, bool f16) {
    return f16 ? pack_f16x2(lo, hi) : pack_bf16x2(lo, hi);
}
__device__ __forceinline__ float out_lo(uint32_t w, bool f16) { return f16 ? f16_lo(w) : bf16_lo(w); }
__device__ __forceinline__ float out_hi(uint32_t w, bool f16) { return f16 ? f16_hi(w) : bf16_hi(w); }

__device__ __forceinline__ float round_to_bf16(float f) {
    return __uint_as_float(f32_to_bf16_bits(f) << 16);
}

// Maximum of two magnitudes (non-negative floats, a NaN among them positive)
// that keeps a NaN, as torch's amax does: the bits of a magnitude order like
// its value, and a positive NaN's bits lie above those of +inf.  (fmaxf
// returns the other operand when one is a NaN.)
__device__ __forceinline__ float mag_max(float a, float b) {
    const uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
    return __uint_as_float(x > y ? x : y);
}

// Wavefront-wide maximum of a magnitude (64 lanes, butterfly; NaN kept).
__device__ __forceinline__ float wave_max(float v) {
    uint32_t b = __float_as_uint(v);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)b, off, 64);
        b = b > o ? b : o;
    }
    return __uint_as_float(b);
}

// torch.clamp(v, -448, 448), which leaves a NaN as it is.  (v_med3_f32 alone
// would not: with a NaN operand it returns the least of the other two, -448.)
__device__ __forceinline__ float clamp_e4m3(float v) {
    const float c = __builtin_amdgcn_fmed3f(v, -kE4M3Max, kE4M3Max);
    return v == v ? c : v;
}

// Two binary32 values (already clamped to +-448) -> two e4m3fn codes in the
// low 16 bits.  gfx950's v_cvt_pk_fp8_f32 produces OCP e4m3fn with round to
// nearest even; the test suite compares it with the oracle over every bf16
// value.
__device__ __forceinline__ uint32_t cvt_e4m3x2(float a, float b) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

// Buffer resource over [base, base + bytes): loads at offsets >= bytes return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Buffer descriptor of an operand region (4 SGPRs): base, stride 0, size in
// bytes (offsets at or beyond it read as zero), raw-buffer format word.
struct CopySrc {
    v4i d;
    __device__ __forceinline__ CopySrc(const void* base, uint32_t bytes) {
        const uint64_t b = (uint64_t)base;
        d = v4i{__builtin_amdgcn_readfirstlane((int)(uint32_t)b),
                __builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32) & 0xFFFF),
                __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
    }
};

// One wave-wide 16-byte-per-lane copy global -> LDS (buffer_load_dwordx4 ...
// lds): lane L's 16 bytes at src + voff land at LDS byte lds_base + 16 L.
// Issued as inline asm so the compiler's wait-count pass, which cannot tell
// that the ring buffer being filled differs from the one being read, does not
// insert a vmcnt(0) before every LDS read; the kernel waits for its copies
// explicitly (wait_vmcnt + ring_barrier).  M0 carries the LDS base; nothing
// else in these kernels uses M0.
__device__ __forceinline__ void copy16(const CopySrc& src, uint32_t lds_base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(src.d)
                 : "memory");
}


}  // namespace h3q
