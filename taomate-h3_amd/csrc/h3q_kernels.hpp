// Host-side launchers of the gfx950 kernels (internal to the library; the
// public C ABI is include/taomate_h3_amd.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace h3q {

hipError_t launch_quant_rows(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, int fmt, int rounding,
                             uint8_t* q, int64_t ldq, float* scales, hipStream_t st);

int64_t tensor_quant_parts(int64_t rows, int64_t k);

hipError_t launch_quant_tensor_e4m3(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k,
                                    const float* static_scale, float* partial, uint8_t* q, int64_t ldq,
                                    float* scale_out, hipStream_t st);

// Operand kinds of the MFMA GEMM.
enum OpKind : int { kOpE4M3 = 0, kOpInt8 = 1, kOpBF16 = 2 };

struct GemmArgs {
    const void* a;          // [m, k] codes (or bf16), row-major, lda bytes between rows
    const void* b;          // [n, k] codes (or bf16), row-major, ldb bytes between rows
    int64_t lda, ldb;       // in BYTES
    int64_t m, n, k;        // k in elements
    const float* a_scale;   // [m] or [1]
    const float* b_scale;   // [n] or [1]
    int a_scale_per_row;
    int b_scale_per_col;
    const uint16_t* bias;   // bf16 [n] or null
    const uint16_t* lora_t; // bf16 [m, r] or null (x @ lora_a^T)
    const uint16_t* lora_b; // bf16 [n, r]
    int64_t ldt, ldlb;      // in elements
    int64_t lora_rank;
    float lora_scale;
    void* out;              // bf16 [m, n] or int32 [m, n]
    int64_t ldo;            // in elements
    int out_vec;            // ldo % 4 == 0, n % 4 == 0 and out 16-byte aligned: 4 columns per store
};

// out = epilogue(A @ B^T).  kind: kOpE4M3 / kOpInt8 scaled to bf16 (with
// optional bias and LoRA); raw_i32: int8 accumulators written as int32;
// kOpBF16: plain bf16 GEMM (LoRA down-projection).
hipError_t launch_gemm(int kind, bool raw_i32, const GemmArgs& args, hipStream_t st);

}  // namespace h3q
