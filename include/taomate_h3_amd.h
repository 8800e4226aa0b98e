/*
 * taomate_h3_amd -- C ABI of the MI355X (gfx950) quantized-linear library.
 *
 * Drop-in native boundary for TaoMate-H3's W8A8 linear path.  Every entry
 * point is stateless and reentrant: it takes raw device pointers, element or
 * byte strides, sizes and a hipStream_t (passed as void*; NULL = the legacy
 * default stream), enqueues its kernels on that stream and returns without
 * synchronising.  Nothing here allocates device memory; buffers belong to the
 * caller.  A non-zero return is an error code; h3q_last_error() then returns
 * a message (thread-local, valid until the next call on the same thread).
 * Argument errors are detected on the host before any launch.
 *
 * Data conventions: bf16 and e4m3fn values are raw bit patterns (uint16_t /
 * uint8_t); matrices are row-major with the given leading dimension.
 */
#ifndef TAOMATE_H3_AMD_H
#define TAOMATE_H3_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Code formats. */
#define H3Q_FMT_E4M3FN 0 /* OCP float8 e4m3fn, largest finite 448 */
#define H3Q_FMT_INT8 1   /* symmetric int8 */
#define H3Q_OUT_F16 0x100 /* h3q_scaled_mm format flag: binary16 output and bias */

/* Rounding forms of the per-row quantizer. */
#define H3Q_ROUND_DIV 0     /* q = round(x / s), s = max(amax * RN(1/L), 1e-12)  (reference weight quantizer) */
#define H3Q_ROUND_RCP_MUL 1 /* q = sat8(rint(x * (127 / amax))), s = amax / 127  (vLLM dynamic int8) */

/* Scale granularities of the scaled GEMM. */
#define H3Q_SCALE_PER_TENSOR 0 /* one fp32 value */
#define H3Q_SCALE_PER_ROW 1    /* a: one per token (row of A); b: one per output channel (row of B) */

/* Operand layouts of the scaled GEMM. */
#define H3Q_LAYOUT_ROWS 0  /* row-major [rows, k] with a leading dimension */
#define H3Q_LAYOUT_TILED 1 /* 16-row x 128-byte tiles in MFMA fragment order (see h3q_quant_rows_tiled) */

/* Status codes. */
#define H3Q_OK 0
#define H3Q_ERR_INVALID 1     /* bad argument (checked before any launch) */
#define H3Q_ERR_UNSUPPORTED 2 /* valid request this build does not implement */
#define H3Q_ERR_HIP 3         /* the HIP runtime refused a launch */

/* Library version (major * 10000 + minor * 100 + patch). */
int h3q_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* h3q_last_error(void);

/*
 * Per-row dynamic quantization of a bf16 matrix x [rows, cols] (leading
 * dimension ldx elements) into codes [rows, cols] (leading dimension ldq
 * bytes) and fp32 scales [rows].
 *
 *   format=E4M3FN, rounding=DIV : s = max(amax*RN(1/448), 1e-12), q = e4m3(clamp(x/s, +-448))
 *   format=INT8,   rounding=DIV : s = max(amax*RN(1/127), 1e-12), q = clamp(rne(x/s), +-127)
 *   format=INT8,   rounding=RCP_MUL : s = amax/127, q = sat8(rne(x * (127/amax))), zero row -> 0
 *
 * DIV scales are the reference's torch.clamp(amax.float() / L, min=1e-12) as
 * PyTorch evaluates it on the GPU (a tensor divided by a Python scalar is a
 * multiply by the binary32 reciprocal of the scalar); x/s is IEEE division.
 *
 * Replaces vLLM torch.ops._C.dynamic_scaled_int8_quant(out, in, scales, None)
 * (called at H3/inference/w8a8.py:178 and, allocating, :212) with RCP_MUL,
 * and the weight quantizer _quantize_weight (H3/inference/w8a8.py:57-63;
 * FL/inference/w8a8.py:242-257) with INT8+DIV, applied to any row range so the
 * 8 MiB streamed loader (H3/inference/w8a8.py:98-133) keeps its chunking.
 * E4M3FN+DIV is the per-token / per-output-channel FP8 quantizer.
 */
int h3q_quant_rows(const void* x, int64_t rows, int64_t cols, int64_t ldx, int format, int rounding,
                   void* codes, int64_t ldq, float* scales, void* stream);

/*
 * Tiled layout (H3Q_LAYOUT_TILED), the packed weight format of the GEMMs.
 * A matrix of `rows` x `cols` codes (cols % 128 == 0) is stored as
 * ceil(rows / 16) x (cols / 128) blocks of 2048 bytes; block (b, s) holds rows
 * 16 b .. 16 b + 15, bytes 128 s .. 128 s + 127 at byte offset
 * (b * cols / 128 + s) * 2048, and inside it code (r, k) sits at
 *   (k % 32 / 16) * 1024 + (r % 16 + 16 * (k % 128 / 32)) * 16 + k % 16,
 * i.e. the operand order of the 16 x 16 x 128 matrix instruction: each half of
 * a lane's 32-byte fragment is one 16-byte slot, a block reads as two
 * contiguous 1 KiB wavefront loads.  Rows past `rows` up to the next multiple
 * of 16 may hold anything: a row of A past m only feeds output rows past m,
 * a row of B past n only output columns past n, and those are not stored.
 * h3q_tiled_bytes() gives the size (0 if cols % 128 != 0).
 *
 * h3q_quant_rows_tiled quantizes rows [row0, row0 + rows) of such a matrix,
 * from x [rows, cols] (ldx elements), exactly as h3q_quant_rows does (same
 * format / rounding semantics and scales, scales[i] for row row0 + i), and
 * writes the codes into their tiled positions.  It is the offline weight
 * quantize-and-pack step: called per row chunk it serves the 8 MiB streamed
 * loader of H3/inference/w8a8.py:98-133 (chunks of any row count).
 */
int64_t h3q_tiled_bytes(int64_t rows, int64_t cols);
int h3q_quant_rows_tiled(const void* x, int64_t rows, int64_t cols, int64_t ldx, int format, int rounding,
                         int64_t row0, void* codes_tiled, float* scales, void* stream);

/*
 * Per-tensor e4m3fn quantization with a bf16 intermediate:
 *   s = static_scale ? *static_scale : max(amax(|x|) * RN(1/448), 1e-12)
 *   q = e4m3(clamp(bf16(x / s), +-448));  *scale_out = s
 * Replaces quantize_fp8_e4m3_dynamic / quantize_fp8_e4m3
 * (FL/inference/fused_kernels.py:771-820) and the per-tensor FP8 weight
 * quantizer (FL/inference/fp8.py:259-263, :107-113).  `partial` is caller
 * workspace of h3q_quant_tensor_workspace_floats(rows, cols) floats (unused
 * when static_scale is given).  Two kernels: partial maxima, then quantize.
 */
int64_t h3q_quant_tensor_workspace_floats(int64_t rows, int64_t cols);
int h3q_quant_tensor_e4m3(const void* x, int64_t rows, int64_t cols, int64_t ldx, const float* static_scale,
                          float* partial, void* codes, int64_t ldq, float* scale_out, void* stream);

/*
 * Per-tensor e4m3fn of a bf16, fp16 or fp32 tensor (dtype: H3Q_DTYPE_*), in
 * either form of the reference (form):
 *   H3Q_QUOTIENT_EAGER   torch's clamp(x / s, -448, 448) evaluated in x's
 *                        dtype (FL/inference/fused_kernels.py:773,
 *                        FL/inference/fp8.py:107-113): divisor and quotient
 *                        rounded to bf16 / fp16 for those inputs, neither
 *                        for fp32;
 *   H3Q_QUOTIENT_TRITON  bf16(x / s) with the fp32 divisor, whatever the
 *                        input (FL/inference/fused_kernels.py:240-246).
 * The scale, workspace and results are those of h3q_quant_tensor_e4m3 (bf16
 * input takes the same kernels).  A quotient 0 / 0 (fp16 divisor rounded to
 * zero, i.e. an all-zero fp16 tensor in the eager form) gives the NaN code
 * 0x7F, as the reference does.  fp16 and fp32 inputs
 * run an elementwise kernel.
 */
#define H3Q_DTYPE_BF16 0
#define H3Q_DTYPE_F16 1
#define H3Q_DTYPE_F32 2
#define H3Q_QUOTIENT_EAGER 0
#define H3Q_QUOTIENT_TRITON 1
int h3q_quant_tensor_e4m3_typed(const void* x, int dtype, int form, int64_t rows, int64_t cols, int64_t ldx,
                                const float* static_scale, float* partial, void* codes, int64_t ldq,
                                float* scale_out, void* stream);

/*
 * h3q_quant_tensor_e4m3 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.  The
 * partial maxima go to a static 4 KiB device array of the library (1024
 * floats, one copy per GPU, held until the process ends; the current
 * device's copy is used, so make the stream's device current), which holds every
 * partial of any shape the kernels launch; a request needing more is refused
 * with H3Q_ERR_UNSUPPORTED.  Nothing is allocated and nothing needs clearing.
 * All calls on one GPU share the array: calls that overlap in time on one GPU
 * (different streams, or other threads) race and must be serialised by the
 * caller.  Results are those of h3q_quant_tensor_e4m3 bit for bit.
 */
int h3q_quant_tensor_e4m3_noalloc(const void* x, int64_t rows, int64_t cols, int64_t ldx, const float* static_scale,
                                  void* codes, int64_t ldq, float* scale_out, void* stream);

/*
 * The same quantizer with the quotient bf16(x / bf16(s)) (IEEE division by the
 * scale rounded to bf16), *scale_out = s unchanged: the reference's eager
 * expression clamp(value / scale, +-448).to(float8_e4m3fn) as torch evaluates
 * it on the GPU, where a bf16 tensor divided by a 0-dim fp32 tensor computes
 * in bf16 and casts the divisor to bf16 (measured on MI355X).  The reference
 * takes this form for its FP8 weight conversions (FL/inference/fp8.py:259-263,
 * :107-113) and for activations when its Triton kernels are not enabled
 * (FL/inference/fused_kernels.py:771-795); h3q_quant_tensor_e4m3 is the form
 * of its Triton kernels (:230-247, fp32 divisor).
 */
int h3q_quant_tensor_e4m3_bf16_divisor(const void* x, int64_t rows, int64_t cols, int64_t ldx,
                                       const float* static_scale, float* partial, void* codes, int64_t ldq,
                                       float* scale_out, void* stream);

/*
 * Fused SwiGLU, optionally with the per-token quantization of the result:
 *   x: bf16 [rows, 2 * half] (leading dimension ldx), each row [gate | up]
 *   y = bf16(bf16(gate / (1 + exp(-gate))) * up)           bf16 [rows, half]
 * to out (leading dimension ldo; NULL for none) and / or codes [rows, half]
 * (ldq bytes) + fp32 scales [rows] in the format / rounding of
 * h3q_quant_rows.  Replaces fused_swiglu (H3/inference/fused_kernels.py:240-261,
 * 663-677) and the eager F.silu(gate) * up (H3/model/layers.py:469-479) that
 * produce the fc2 input, with the next W8A8 linear's act-quant folded in.  exp
 * is computed from IEEE multiply-adds (within 1 ulp of a correctly rounded
 * exp); the division and product are IEEE.  half % 8 == 0, half <= 16384,
 * 16-byte aligned x / out, strides multiples of 8 elements.
 */
int h3q_swiglu_quant(const void* x, int64_t ldx, int64_t rows, int64_t half, void* out, int64_t ldo, int format,
                     int rounding, void* codes, int64_t ldq, float* scales, void* stream);

/*
 * Per-(batch, head) e4m3fn quantization of attention operands:
 *   x: contiguous bf16 [batch, seq, heads, head_dim]
 *   scales[b, h] = max(amax_{s,d}(|x[b, s, h, d]|) * RN(1/448), 1e-12)   (fp32 [batch, heads])
 *   codes[b, s, h, d] = e4m3(clamp(x / scales[b, h], +-448))   (fp32 quotient, no bf16 intermediate)
 * Replaces quantize_fp8_e4m3_per_head (FL/inference/fused_kernels.py:823-877;
 * Triton :175-227, :250-273), called for the FP8 attention inputs at
 * FL/streaming/attention_hook.py:1018-1043 and FL/streaming/cache.py:838-853.
 * `partial` is caller workspace of
 * h3q_quant_per_head_workspace_floats(batch, seq, heads, head_dim) floats.
 * batch == 0 or heads == 0 is a no-op; seq == 0 or head_dim == 0 is
 * H3Q_ERR_INVALID (an empty reduction, as torch's amax); heads <= 4096.
 * head_dim % 8 == 0 with a 16-byte aligned x and 8-byte aligned codes takes
 * the vector path; anything else runs element by element.  Two kernels:
 * per-chunk head maxima, then fold + quantize.
 */
int64_t h3q_quant_per_head_workspace_floats(int64_t batch, int64_t seq, int64_t heads, int64_t head_dim);
int h3q_quant_per_head_e4m3(const void* x, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                            float* partial, void* codes, float* scales, void* stream);

/*
 * Scaled GEMM with fused epilogue:
 *   out[m, n] = bf16( a_scale[m] * (b_scale[n] * float(sum_k a[m, k] * b[n, k])) [+ bias[n]]
 *                     [+ lora_scale * sum_r lora_t[m, r] * lora_b[n, r]] )
 * a: codes [m, k] (lda bytes), b: weight codes [n, k] (ldb bytes, the
 * nn.Linear layout, i.e. cutlass_scaled_mm's B = weight.t()), format E4M3FN
 * or INT8 for both; format | H3Q_OUT_F16 makes out and bias IEEE binary16
 * (one rounding of the fp32 result, torch._scaled_mm(out_dtype=float16),
 * FL/inference/fp8.py:135-143) instead of bf16 (not with LoRA).  a_layout / b_layout:
 * H3Q_LAYOUT_ROWS, or H3Q_LAYOUT_TILED (k % 128 == 0; the leading dimension
 * is then ignored; tiled activations for m <= 128 without LoRA, for m > 128
 * with or without it, given k >= 256, n and ldo multiples of 8 and a 16-byte
 * aligned bf16 out).  Tiled weights are the
 * fast format for every m (with few rows the GEMM streams them from HBM in
 * 1 KiB loads).  a_scale_kind / b_scale_kind: H3Q_SCALE_PER_ROW or
 * H3Q_SCALE_PER_TENSOR.  bias: bf16 [n] or NULL (added as one fused
 * multiply-add: fma(a_scale, b_scale * acc, bias)).  lora_t: bf16 [m, rank]
 * (ldt elements) = x @ lora_a^T, lora_b: bf16 [n, rank] (ldlb elements), or
 * both NULL; rank <= 128 and a multiple of 8.  out: bf16 [m, n] (ldo elements).
 * Requires k % 16 == 0, lda and ldb multiples of 16 bytes, 16-byte aligned a/b.
 * Replaces vLLM cutlass_scaled_mm (H3/inference/w8a8.py:179-186, :213-219)
 * and torch._scaled_mm (FL/distributed/linear.py:92-100; FL/inference/fp8.py:135-143)
 * plus the LoRA side branch (H3/inference/lora_checkpoint.py:196-205).
 */
int h3q_scaled_mm(int format, const void* a, int64_t lda, int a_layout, const float* a_scale, int a_scale_kind,
                  const void* b, int64_t ldb, int b_layout, const float* b_scale, int b_scale_kind, const void* bias,
                  const void* lora_t, int64_t ldt, const void* lora_b, int64_t ldlb, int64_t lora_rank,
                  float lora_scale, void* out, int64_t ldo, int64_t m, int64_t n, int64_t k, void* stream);

/*
 * Raw int32 accumulators of the int8 GEMM: out[m, n] = sum_k a[m, k] * b[n, k]
 * (a [m, k], b [n, k] int8; out int32, ldo elements).  Exposes the integer
 * core of cutlass_scaled_mm (H3/inference/w8a8.py:179-186) for bit-exact
 * checks.  Same layout requirements as h3q_scaled_mm.
 */
int h3q_gemm_i8_i32(const void* a, int64_t lda, const void* b, int64_t ldb, void* out, int64_t ldo, int64_t m,
                    int64_t n, int64_t k, void* stream);

/*
 * LoRA down-projection t = bf16(x @ lora_a^T): x bf16 [m, k] (ldx elements),
 * lora_a bf16 [rank, k] (lda elements), t bf16 [m, rank] (ldt elements).
 * The first F.linear of H3/inference/lora_checkpoint.py:197-199, whose bf16
 * result feeds h3q_scaled_mm's fused LoRA epilogue.  k % 8 == 0.
 */
int h3q_lora_down(const void* x, int64_t ldx, const void* lora_a, int64_t lda, void* t, int64_t ldt, int64_t m,
                  int64_t k, int64_t rank, void* stream);

/*
 * The same product split over K when x has few rows (below 128 blocks of 96):
 * each K slice's binary32 partial goes to the caller's workspace, then the
 * slices are summed in order and rounded once to bf16 (within the same error
 * bound as h3q_lora_down; deterministic).  h3q_lora_down_workspace_bytes gives
 * the bytes needed (0: the call does not split and needs no workspace); a
 * smaller workspace is an error.  No counterpart in the reference: the
 * reference's F.linear (H3/inference/lora_checkpoint.py:197-199) leaves this
 * to the BLAS library; the split keeps the H3 shapes (M = 592 .. 6224 tokens)
 * from running on a few dozen workgroups.
 */
int64_t h3q_lora_down_workspace_bytes(int64_t m, int64_t k, int64_t rank);
int h3q_lora_down_ws(const void* x, int64_t ldx, const void* lora_a, int64_t lda, void* t, int64_t ldt, int64_t m,
                     int64_t k, int64_t rank, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Fused RMSNorm + AdaLN modulate + per-token quantization: the producer of the
 * QKV input of a DiT block, fused_rms_norm_modulate
 * (H3/inference/fused_kernels.py:287-317 kernel, 700-730 wrapper), with the
 * activation quantizer of the following W8A8 linear folded in.  For each row r
 * (t = indices[r], a row of the [T, table_stride] scale / shift tables):
 *   rs = 1 / sqrt(sum_k v[k]^2 / cols + eps)            (binary32; see below)
 *   n  = bf16((v[k] * rs) * weight[k])
 *   y  = bf16(bf16(n * bf16(1 + scale[t, k])) + shift[t, k])
 * y goes to out (bf16, ldo elements) when out is not NULL; when codes is not
 * NULL, y is quantized per row exactly as h3q_quant_rows(format, rounding)
 * does (codes row-major with ldq bytes, scales[r]).  At least one of out and
 * codes must be given.  The sum of squares is taken in a fixed order (lane l
 * of a 64-lane group adds elements 8 (l + 64 i) + e in ascending (i, e), then
 * a butterfly xor 32, 16, ..., 1 adds the lane sums) and rs is an IEEE square
 * root followed by an IEEE division, so results are reproducible on a CPU;
 * the reference's Triton rsqrt may differ in the last bits.
 * bf16 tensors: value [rows, cols] (ldv), weight [cols], tables; indices
 * int64 [rows] (not range-checked, as in the reference).  cols % 8 == 0,
 * cols <= 8192, strides multiples of 8 elements, bf16 pointers 16-byte
 * aligned, codes 8-byte aligned.
 */
int h3q_rms_norm_modulate_quant(const void* value, int64_t ldv, const void* weight, const void* scale,
                                const void* shift, int64_t table_stride, const int64_t* indices, int64_t rows,
                                int64_t cols, float eps, void* out, int64_t ldo, int format, int rounding, void* codes,
                                int64_t ldq, float* scales, void* stream);

/*
 * The fc1-input producer fused_residual_gate_rms_norm_modulate
 * (H3/inference/fused_kernels.py:319-357 kernel, 733-773 wrapper) with the
 * same quantizer folded in: hidden = bf16(residual + bf16(gate[t, k] *
 * branch)) is stored (ldh elements) and then normalized, modulated and
 * quantized as in h3q_rms_norm_modulate_quant.
 */
int h3q_residual_gate_rms_norm_modulate_quant(const void* residual, int64_t ldr, const void* branch, int64_t ldb,
                                              const void* gate, const void* weight, const void* scale,
                                              const void* shift, int64_t table_stride, const int64_t* indices,
                                              int64_t rows, int64_t cols, float eps, void* hidden, int64_t ldh,
                                              void* out, int64_t ldo, int format, int rounding, void* codes,
                                              int64_t ldq, float* scales, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TAOMATE_H3_AMD_H */
