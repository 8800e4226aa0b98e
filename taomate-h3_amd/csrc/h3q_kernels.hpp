// Host-side launchers of the gfx950 kernels (internal to the library; the
// public C ABI is include/taomate_h3_amd.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace h3q {

hipError_t launch_quant_rows(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, int fmt, int rounding,
                             uint8_t* q, int64_t ldq, float* scales, hipStream_t st);

// Rows [row0, row0 + rows) of a K-column matrix into the tiled weight layout
// (K % 128 == 0; see code_offset in act_quant.hip); scales[i] is row row0 + i.
hipError_t launch_quant_rows_tiled(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k, int fmt, int rounding,
                                   uint8_t* q_tiled, int64_t row0, float* scales, hipStream_t st);

int64_t tensor_quant_parts(int64_t rows, int64_t k);

// Device address of the per-tensor quantizer's static scratch on the current
// device (kTensorScratchFloats floats, looked up once per device).
constexpr int64_t kTensorScratchFloats = 1024;
hipError_t tensor_scratch(float** out);

// Input types of the typed per-tensor quantizer (mirrored by include/taomate_h3_amd.h).
enum TensorIn : int { kInBF16 = 0, kInF16 = 1, kInF32 = 2 };

// Per-tensor e4m3 of bf16 / fp16 / fp32 input; eager: torch's clamp(x / s) in
// x's dtype, else the fp32-divisor quotient rounded to bf16.  bf16 input runs
// the vector kernels of launch_quant_tensor_e4m3.
hipError_t launch_quant_tensor_e4m3_typed(const void* x, int in, bool eager, int64_t ldx, int64_t rows, int64_t k,
                                          const float* static_scale, float* partial, uint8_t* q, int64_t ldq,
                                          float* scale_out, hipStream_t st);

hipError_t launch_quant_tensor_e4m3(const uint16_t* x, int64_t ldx, int64_t rows, int64_t k,
                                    const float* static_scale, bool bf16_divisor, float* partial, uint8_t* q,
                                    int64_t ldq, float* scale_out, hipStream_t st);

// Fused SwiGLU (+ per-token quantization): rows of x are [gate (half) | up
// (half)] bf16; y = bf16(bf16(silu(gate)) * up) to out (optional, [rows, half])
// and / or its codes + scales.  half % 8 == 0, half <= kSwigluMaxHalf, 16-byte
// aligned rows.
struct SwigluQuantArgs {
    const uint16_t* x;
    int64_t ldx, rows;
    int half;
    uint16_t* out;
    int64_t ldo;
    uint8_t* codes;
    int64_t ldq;
    float* scales;
};
constexpr int kSwigluMaxHalf = 16384;
hipError_t launch_swiglu_quant(const SwigluQuantArgs& a, int fmt, int rounding, hipStream_t st);

// Per-(batch, head) e4m3fn quantization of a contiguous [batch, seq, heads,
// head_dim] bf16 tensor: codes of the same shape, scales [batch, heads].
// partial holds per_head_quant_parts(...) floats.
constexpr int64_t kMaxHeads = 4096;
int64_t per_head_quant_parts(int64_t batch, int64_t seq, int64_t heads, int64_t head_dim);
hipError_t launch_quant_per_head_e4m3(const uint16_t* x, int64_t batch, int64_t seq, int64_t heads,
                                      int64_t head_dim, float* partial, uint8_t* q, float* scales,
                                      hipStream_t st);

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
    int a_tiled, b_tiled;   // operand stored in the tiled layout (k % 128 == 0; rows padded to 16 with zeros)
    int out_f16;            // scaled output and bias are IEEE binary16 instead of bf16
    int64_t kt_split;       // LoRA down-projection split over K: k-tiles per slice (blockIdx.y), 0: no split
};

// out = epilogue(A @ B^T).  kind: kOpE4M3 / kOpInt8 scaled to bf16 (with
// optional bias and LoRA); raw_i32: int8 accumulators written as int32;
// kOpBF16: plain bf16 GEMM (LoRA down-projection).
hipError_t launch_gemm(int kind, bool raw_i32, const GemmArgs& args, hipStream_t st);

// LoRA down-projection t = bf16(x @ lora_a^T) (kind kOpBF16, n = rank).  With
// few rows the call is split over K: each slice's binary32 partial goes to
// the workspace and a second kernel sums the slices in order and rounds.
// lora_down_workspace_bytes gives the bytes that split needs (0: no split).
int64_t lora_down_workspace_bytes(int64_t m, int64_t k, int64_t rank);
hipError_t launch_lora_down(const GemmArgs& args, void* workspace, int64_t workspace_bytes, hipStream_t st);

// Persistent four-wave GEMM for large M (gemm_w4.hip): scaled e4m3 / int8 ->
// bf16 (or binary16) with optional bias and rank <= 128 LoRA; row-major or
// tiled A and B; k % 128 == 0, k >= 256, n % 8 == 0, ldo % 8 == 0, 16-byte
// aligned output, m > kSkinnyMaxM.
// launch_gemm routes there itself when w4_supported() holds.
bool w4_supported(const GemmArgs& a);
hipError_t launch_gemm_w4(int kind, const GemmArgs& a, hipStream_t st);

// Weight-streaming GEMM for M <= kSkinnyMaxM activation rows (scaled e4m3 /
// int8 to bf16, optional bias, no LoRA).  launch_gemm routes there itself.
constexpr int64_t kSkinnyMaxM = 128;
bool skinny_supported(const GemmArgs& a);
hipError_t launch_gemm_skinny(int kind, const GemmArgs& a, hipStream_t st);

// Fused RMSNorm + AdaLN modulate (+ residual gate) + per-token quantization
// (norm_quant.hip).  All bf16 tensors are row-major with element strides;
// tables are [T, table_stride] and row r uses table row indices[r].
struct NormQuantArgs {
    const uint16_t* value;   // [rows, cols]; with the residual gate: the residual
    const uint16_t* branch;  // residual gate only: [rows, cols]
    const uint16_t* gate;    // residual gate only: gate table
    const uint16_t* weight;  // [cols] RMSNorm weight
    const uint16_t* scale;   // modulate scale table
    const uint16_t* shift;   // modulate shift table
    const int64_t* indices;  // [rows]
    int64_t ldv, ldb, table_stride, rows;
    int cols;                // multiple of 8, at most 8192
    float eps;
    uint16_t* hidden;        // residual gate only: [rows, cols] out
    int64_t ldh;
    uint16_t* out;           // [rows, cols] bf16 modulated output, or null
    int64_t ldo;
    uint8_t* codes;          // [rows, cols] codes (row-major, ldq bytes), or null
    int64_t ldq;
    float* scales;           // [rows] per-token scales (with codes)
};
constexpr int kNormQuantMaxCols = 8192;
hipError_t launch_norm_modulate_quant(const NormQuantArgs& a, bool resid, int fmt, int rounding, hipStream_t st);

}  // namespace h3q
