// C ABI entry points (include/taomate_h3_amd.h): host-side argument checks,
// then one or two kernel launches on the caller's stream.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/taomate_h3_amd.h"
#include "h3q_kernels.hpp"

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_error[0] = '\0';
    return H3Q_OK;
}

int check_launch(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(H3Q_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int h3q_version(void) { return 200; }

__attribute__((visibility("default"))) const char* h3q_last_error(void) { return g_error; }

__attribute__((visibility("default"))) int h3q_quant_rows(const void* x, int64_t rows, int64_t cols, int64_t ldx,
                                                          int format, int rounding, void* codes, int64_t ldq,
                                                          float* scales, void* stream) {
    if (rows < 0 || cols < 0) return fail(H3Q_ERR_INVALID, "h3q_quant_rows: negative shape [%lld, %lld]",
                                          (long long)rows, (long long)cols);
    if (format != H3Q_FMT_E4M3FN && format != H3Q_FMT_INT8)
        return fail(H3Q_ERR_INVALID, "h3q_quant_rows: unknown format %d", format);
    if (rounding != H3Q_ROUND_DIV && rounding != H3Q_ROUND_RCP_MUL)
        return fail(H3Q_ERR_INVALID, "h3q_quant_rows: unknown rounding %d", rounding);
    if (format == H3Q_FMT_E4M3FN && rounding != H3Q_ROUND_DIV)
        return fail(H3Q_ERR_UNSUPPORTED, "h3q_quant_rows: e4m3fn codes use the division form only");
    if (ldx < cols || ldq < cols) return fail(H3Q_ERR_INVALID, "h3q_quant_rows: leading dimension below cols");
    if (rows == 0) return ok();
    if (!x || !codes || !scales) return fail(H3Q_ERR_INVALID, "h3q_quant_rows: null pointer");
    if (cols == 0) return fail(H3Q_ERR_INVALID, "h3q_quant_rows: zero-width rows have no scale");
    return check_launch(h3q::launch_quant_rows((const uint16_t*)x, ldx, rows, cols, format, rounding,
                                               (uint8_t*)codes, ldq, scales, (hipStream_t)stream),
                        "h3q_quant_rows");
}

// Shared checks of the fused norm / modulate / quantize entry points.
static int check_norm_quant(const char* who, int64_t rows, int64_t cols, int64_t table_stride, const void* weight,
                            const void* scale, const void* shift, const int64_t* indices, const void* out,
                            int64_t ldo, int format, int rounding, const void* codes, int64_t ldq,
                            const float* scales) {
    if (rows < 0 || cols <= 0) return fail(H3Q_ERR_INVALID, "%s: bad shape [%lld, %lld]", who, (long long)rows, (long long)cols);
    if (cols % 8) return fail(H3Q_ERR_UNSUPPORTED, "%s: cols=%lld must be a multiple of 8", who, (long long)cols);
    if (cols > h3q::kNormQuantMaxCols)
        return fail(H3Q_ERR_UNSUPPORTED, "%s: cols=%lld above %d", who, (long long)cols, h3q::kNormQuantMaxCols);
    if (table_stride < cols || table_stride % 8)
        return fail(H3Q_ERR_INVALID, "%s: table stride %lld must be >= cols and a multiple of 8", who,
                    (long long)table_stride);
    if (!out && !codes) return fail(H3Q_ERR_INVALID, "%s: neither a bf16 output nor codes requested", who);
    if (out && (ldo < cols || ldo % 8)) return fail(H3Q_ERR_INVALID, "%s: bad output stride %lld", who, (long long)ldo);
    if (codes) {
        if (format != H3Q_FMT_E4M3FN && format != H3Q_FMT_INT8)
            return fail(H3Q_ERR_INVALID, "%s: unknown format %d", who, format);
        if (rounding != H3Q_ROUND_DIV && rounding != H3Q_ROUND_RCP_MUL)
            return fail(H3Q_ERR_INVALID, "%s: unknown rounding %d", who, rounding);
        if (format == H3Q_FMT_E4M3FN && rounding != H3Q_ROUND_DIV)
            return fail(H3Q_ERR_UNSUPPORTED, "%s: e4m3fn codes use the division form only", who);
        if (ldq < cols || ldq % 8) return fail(H3Q_ERR_INVALID, "%s: bad codes stride %lld", who, (long long)ldq);
        if (!scales) return fail(H3Q_ERR_INVALID, "%s: codes need a scales pointer", who);
        if (!aligned(codes, 8)) return fail(H3Q_ERR_INVALID, "%s: codes must be 8-byte aligned", who);
    }
    if (rows > 0 && (!weight || !scale || !shift || !indices)) return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    if (!aligned(weight, 16) || !aligned(scale, 16) || !aligned(shift, 16) || (out && !aligned(out, 16)))
        return fail(H3Q_ERR_INVALID, "%s: bf16 operands must be 16-byte aligned", who);
    return H3Q_OK;
}

__attribute__((visibility("default"))) int h3q_rms_norm_modulate_quant(
    const void* value, int64_t ldv, const void* weight, const void* scale, const void* shift, int64_t table_stride,
    const int64_t* indices, int64_t rows, int64_t cols, float eps, void* out, int64_t ldo, int format, int rounding,
    void* codes, int64_t ldq, float* scales, void* stream) {
    const char* who = "h3q_rms_norm_modulate_quant";
    int rc = check_norm_quant(who, rows, cols, table_stride, weight, scale, shift, indices, out, ldo, format, rounding,
                              codes, ldq, scales);
    if (rc != H3Q_OK) return rc;
    if (ldv < cols || ldv % 8) return fail(H3Q_ERR_INVALID, "%s: bad value stride %lld", who, (long long)ldv);
    if (rows == 0) return ok();
    if (!value || !aligned(value, 16)) return fail(H3Q_ERR_INVALID, "%s: value must be non-null and 16-byte aligned", who);
    h3q::NormQuantArgs a{};
    a.value = (const uint16_t*)value;
    a.ldv = ldv;
    a.weight = (const uint16_t*)weight;
    a.scale = (const uint16_t*)scale;
    a.shift = (const uint16_t*)shift;
    a.table_stride = table_stride;
    a.indices = indices;
    a.rows = rows;
    a.cols = (int)cols;
    a.eps = eps;
    a.out = (uint16_t*)out;
    a.ldo = ldo;
    a.codes = (uint8_t*)codes;
    a.ldq = ldq;
    a.scales = scales;
    return check_launch(h3q::launch_norm_modulate_quant(a, false, format, rounding, (hipStream_t)stream), who);
}

__attribute__((visibility("default"))) int h3q_residual_gate_rms_norm_modulate_quant(
    const void* residual, int64_t ldr, const void* branch, int64_t ldb, const void* gate, const void* weight,
    const void* scale, const void* shift, int64_t table_stride, const int64_t* indices, int64_t rows, int64_t cols,
    float eps, void* hidden, int64_t ldh, void* out, int64_t ldo, int format, int rounding, void* codes, int64_t ldq,
    float* scales, void* stream) {
    const char* who = "h3q_residual_gate_rms_norm_modulate_quant";
    int rc = check_norm_quant(who, rows, cols, table_stride, weight, scale, shift, indices, out, ldo, format, rounding,
                              codes, ldq, scales);
    if (rc != H3Q_OK) return rc;
    if (ldr < cols || ldr % 8 || ldb < cols || ldb % 8 || ldh < cols || ldh % 8)
        return fail(H3Q_ERR_INVALID, "%s: bad residual / branch / hidden stride", who);
    if (rows == 0) return ok();
    if (!residual || !branch || !gate || !hidden) return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    if (!aligned(residual, 16) || !aligned(branch, 16) || !aligned(gate, 16) || !aligned(hidden, 16))
        return fail(H3Q_ERR_INVALID, "%s: bf16 operands must be 16-byte aligned", who);
    h3q::NormQuantArgs a{};
    a.value = (const uint16_t*)residual;
    a.ldv = ldr;
    a.branch = (const uint16_t*)branch;
    a.ldb = ldb;
    a.gate = (const uint16_t*)gate;
    a.weight = (const uint16_t*)weight;
    a.scale = (const uint16_t*)scale;
    a.shift = (const uint16_t*)shift;
    a.table_stride = table_stride;
    a.indices = indices;
    a.rows = rows;
    a.cols = (int)cols;
    a.eps = eps;
    a.hidden = (uint16_t*)hidden;
    a.ldh = ldh;
    a.out = (uint16_t*)out;
    a.ldo = ldo;
    a.codes = (uint8_t*)codes;
    a.ldq = ldq;
    a.scales = scales;
    return check_launch(h3q::launch_norm_modulate_quant(a, true, format, rounding, (hipStream_t)stream), who);
}

__attribute__((visibility("default"))) int64_t h3q_tiled_bytes(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0 || cols % 128) return 0;
    return (rows + 15) / 16 * (cols / 128) * 2048;
}

__attribute__((visibility("default"))) int h3q_quant_rows_tiled(const void* x, int64_t rows, int64_t cols,
                                                                int64_t ldx, int format, int rounding, int64_t row0,
                                                                void* codes_tiled, float* scales, void* stream) {
    const char* who = "h3q_quant_rows_tiled";
    if (rows < 0 || cols <= 0 || row0 < 0)
        return fail(H3Q_ERR_INVALID, "%s: bad shape rows=%lld cols=%lld row0=%lld", who, (long long)rows,
                    (long long)cols, (long long)row0);
    if (cols % 128) return fail(H3Q_ERR_INVALID, "%s: cols=%lld must be a multiple of 128", who, (long long)cols);
    if (format != H3Q_FMT_E4M3FN && format != H3Q_FMT_INT8)
        return fail(H3Q_ERR_INVALID, "%s: unknown format %d", who, format);
    if (rounding != H3Q_ROUND_DIV && rounding != H3Q_ROUND_RCP_MUL)
        return fail(H3Q_ERR_INVALID, "%s: unknown rounding %d", who, rounding);
    if (format == H3Q_FMT_E4M3FN && rounding != H3Q_ROUND_DIV)
        return fail(H3Q_ERR_UNSUPPORTED, "%s: e4m3fn codes use the division form only", who);
    if (ldx < cols) return fail(H3Q_ERR_INVALID, "%s: leading dimension below cols", who);
    if (rows == 0) return ok();
    if (!x || !codes_tiled || !scales) return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    if (!aligned(codes_tiled, 16)) return fail(H3Q_ERR_INVALID, "%s: tiled codes must be 16-byte aligned", who);
    return check_launch(h3q::launch_quant_rows_tiled((const uint16_t*)x, ldx, rows, cols, format, rounding,
                                                     (uint8_t*)codes_tiled, row0, scales, (hipStream_t)stream),
                        who);
}

__attribute__((visibility("default"))) int64_t h3q_quant_tensor_workspace_floats(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0) return 1;
    return h3q::tensor_quant_parts(rows, cols);
}

// in: h3q::TensorIn; eager: torch's clamp(x / s) in x's dtype (for bf16 the
// bf16 divisor), else the fp32 divisor with the quotient rounded to bf16.
static int quant_tensor_e4m3(const char* who, const void* x, int in, int64_t rows, int64_t cols, int64_t ldx,
                             const float* static_scale, bool eager, float* partial, void* codes, int64_t ldq,
                             float* scale_out, void* stream) {
    if (rows <= 0 || cols <= 0) return fail(H3Q_ERR_INVALID, "%s: empty tensor has no amax", who);
    if (ldx < cols || ldq < cols) return fail(H3Q_ERR_INVALID, "%s: leading dimension below cols", who);
    if (!x || !codes || !scale_out || (!static_scale && !partial))
        return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    return check_launch(h3q::launch_quant_tensor_e4m3_typed(x, in, eager, ldx, rows, cols, static_scale, partial,
                                                            (uint8_t*)codes, ldq, scale_out, (hipStream_t)stream),
                        who);
}

__attribute__((visibility("default"))) int h3q_quant_tensor_e4m3(const void* x, int64_t rows, int64_t cols,
                                                                 int64_t ldx, const float* static_scale,
                                                                 float* partial, void* codes, int64_t ldq,
                                                                 float* scale_out, void* stream) {
    return quant_tensor_e4m3("h3q_quant_tensor_e4m3", x, h3q::kInBF16, rows, cols, ldx, static_scale, false, partial,
                             codes, ldq, scale_out, stream);
}

__attribute__((visibility("default"))) int h3q_quant_tensor_e4m3_noalloc(const void* x, int64_t rows,
                                                                         int64_t cols, int64_t ldx,
                                                                         const float* static_scale, void* codes,
                                                                         int64_t ldq, float* scale_out,
                                                                         void* stream) {
    const char* who = "h3q_quant_tensor_e4m3_noalloc";
    if (rows > 0 && cols > 0 && h3q::tensor_quant_parts(rows, cols) > h3q::kTensorScratchFloats)
        return fail(H3Q_ERR_UNSUPPORTED, "%s: %lld partial maxima exceed the %lld-float scratch", who,
                    (long long)h3q::tensor_quant_parts(rows, cols), (long long)h3q::kTensorScratchFloats);
    float* scratch = nullptr;
    if (rows > 0 && cols > 0 && !static_scale) {
        const hipError_t e = h3q::tensor_scratch(&scratch);
        if (e != hipSuccess) return fail(H3Q_ERR_HIP, "%s: scratch address: %s", who, hipGetErrorString(e));
    }
    return quant_tensor_e4m3(who, x, h3q::kInBF16, rows, cols, ldx, static_scale, false, scratch, codes, ldq,
                             scale_out, stream);
}

__attribute__((visibility("default"))) int h3q_quant_tensor_e4m3_bf16_divisor(const void* x, int64_t rows,
                                                                              int64_t cols, int64_t ldx,
                                                                              const float* static_scale,
                                                                              float* partial, void* codes,
                                                                              int64_t ldq, float* scale_out,
                                                                              void* stream) {
    return quant_tensor_e4m3("h3q_quant_tensor_e4m3_bf16_divisor", x, h3q::kInBF16, rows, cols, ldx, static_scale, true,
                             partial, codes, ldq, scale_out, stream);
}

__attribute__((visibility("default"))) int h3q_quant_tensor_e4m3_typed(const void* x, int dtype, int form,
                                                                       int64_t rows, int64_t cols, int64_t ldx,
                                                                       const float* static_scale, float* partial,
                                                                       void* codes, int64_t ldq, float* scale_out,
                                                                       void* stream) {
    const char* who = "h3q_quant_tensor_e4m3_typed";
    if (dtype != H3Q_DTYPE_BF16 && dtype != H3Q_DTYPE_F16 && dtype != H3Q_DTYPE_F32)
        return fail(H3Q_ERR_INVALID, "%s: unknown input dtype %d", who, dtype);
    if (form != H3Q_QUOTIENT_EAGER && form != H3Q_QUOTIENT_TRITON)
        return fail(H3Q_ERR_INVALID, "%s: unknown quotient form %d", who, form);
    const int in = dtype == H3Q_DTYPE_BF16 ? h3q::kInBF16 : dtype == H3Q_DTYPE_F16 ? h3q::kInF16 : h3q::kInF32;
    return quant_tensor_e4m3(who, x, in, rows, cols, ldx, static_scale, form == H3Q_QUOTIENT_EAGER, partial, codes,
                             ldq, scale_out, stream);
}

__attribute__((visibility("default"))) int h3q_swiglu_quant(const void* x, int64_t ldx, int64_t rows, int64_t half,
                                                            void* out, int64_t ldo, int format, int rounding,
                                                            void* codes, int64_t ldq, float* scales, void* stream) {
    const char* who = "h3q_swiglu_quant";
    if (rows < 0 || half <= 0) return fail(H3Q_ERR_INVALID, "%s: bad shape [%lld, 2 x %lld]", who, (long long)rows, (long long)half);
    if (half % 8) return fail(H3Q_ERR_UNSUPPORTED, "%s: half=%lld must be a multiple of 8", who, (long long)half);
    if (half > h3q::kSwigluMaxHalf)
        return fail(H3Q_ERR_UNSUPPORTED, "%s: half=%lld above %d", who, (long long)half, h3q::kSwigluMaxHalf);
    if (ldx < 2 * half || ldx % 8) return fail(H3Q_ERR_INVALID, "%s: bad input stride %lld", who, (long long)ldx);
    if (!out && !codes) return fail(H3Q_ERR_INVALID, "%s: neither a bf16 output nor codes requested", who);
    if (out && (ldo < half || ldo % 8 || !aligned(out, 16)))
        return fail(H3Q_ERR_INVALID, "%s: output needs a stride >= half, a multiple of 8, and 16-byte alignment", who);
    if (codes) {
        if (format != H3Q_FMT_E4M3FN && format != H3Q_FMT_INT8)
            return fail(H3Q_ERR_INVALID, "%s: unknown format %d", who, format);
        if (rounding != H3Q_ROUND_DIV && rounding != H3Q_ROUND_RCP_MUL)
            return fail(H3Q_ERR_INVALID, "%s: unknown rounding %d", who, rounding);
        if (format == H3Q_FMT_E4M3FN && rounding != H3Q_ROUND_DIV)
            return fail(H3Q_ERR_UNSUPPORTED, "%s: e4m3fn codes use the division form only", who);
        if (ldq < half || ldq % 8 || !aligned(codes, 8))
            return fail(H3Q_ERR_INVALID, "%s: codes need a stride >= half, a multiple of 8, and 8-byte alignment", who);
        if (!scales) return fail(H3Q_ERR_INVALID, "%s: codes need a scales pointer", who);
    }
    if (rows == 0) return ok();
    if (!x || !aligned(x, 16)) return fail(H3Q_ERR_INVALID, "%s: x must be non-null and 16-byte aligned", who);
    h3q::SwigluQuantArgs a{};
    a.x = (const uint16_t*)x;
    a.ldx = ldx;
    a.rows = rows;
    a.half = (int)half;
    a.out = (uint16_t*)out;
    a.ldo = ldo;
    a.codes = (uint8_t*)codes;
    a.ldq = ldq;
    a.scales = scales;
    return check_launch(h3q::launch_swiglu_quant(a, format, rounding, (hipStream_t)stream), who);
}

__attribute__((visibility("default"))) int64_t h3q_quant_per_head_workspace_floats(int64_t batch, int64_t seq,
                                                                                   int64_t heads, int64_t head_dim) {
    if (batch <= 0 || seq <= 0 || heads <= 0 || head_dim <= 0 || heads > h3q::kMaxHeads) return 1;
    return h3q::per_head_quant_parts(batch, seq, heads, head_dim);
}

__attribute__((visibility("default"))) int h3q_quant_per_head_e4m3(const void* x, int64_t batch, int64_t seq,
                                                                   int64_t heads, int64_t head_dim, float* partial,
                                                                   void* codes, float* scales, void* stream) {
    const char* who = "h3q_quant_per_head_e4m3";
    if (batch < 0 || seq < 0 || heads < 0 || head_dim < 0) return fail(H3Q_ERR_INVALID, "%s: negative shape", who);
    if (batch == 0 || heads == 0) return H3Q_OK;  // no (batch, head) pair: nothing to reduce or write
    if (seq == 0 || head_dim == 0)
        return fail(H3Q_ERR_INVALID, "%s: empty (seq, head_dim) reduction has no amax", who);
    if (heads > h3q::kMaxHeads)
        return fail(H3Q_ERR_UNSUPPORTED, "%s: heads=%lld above %lld", who, (long long)heads,
                    (long long)h3q::kMaxHeads);
    if (heads * head_dim >= (int64_t(1) << 30) || batch * heads >= (int64_t(1) << 30))
        return fail(H3Q_ERR_UNSUPPORTED, "%s: row or batch x heads above 2^30", who);
    if (!x || !partial || !codes || !scales) return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    if (!aligned(x, 2) || !aligned(scales, 4) || !aligned(partial, 4))
        return fail(H3Q_ERR_INVALID, "%s: misaligned pointer", who);
    return check_launch(h3q::launch_quant_per_head_e4m3((const uint16_t*)x, batch, seq, heads, head_dim, partial,
                                                        (uint8_t*)codes, scales, (hipStream_t)stream),
                        who);
}

static int check_gemm_operands(const char* who, const void* a, int64_t lda, const void* b, int64_t ldb, int64_t m,
                               int64_t n, int64_t k, int64_t elem, bool a_tiled = false, bool b_tiled = false) {
    if (m < 0 || n < 0 || k < 0) return fail(H3Q_ERR_INVALID, "%s: negative shape", who);
    if (k % 16) return fail(H3Q_ERR_INVALID, "%s: k=%lld must be a multiple of 16", who, (long long)k);
    if ((a_tiled || b_tiled) && k % 128)
        return fail(H3Q_ERR_INVALID, "%s: tiled operands need k=%lld to be a multiple of 128", who, (long long)k);
    if ((!a_tiled && lda < k * elem) || (!b_tiled && ldb < k * elem))
        return fail(H3Q_ERR_INVALID, "%s: leading dimension below k", who);
    if ((!a_tiled && lda % 16) || (!b_tiled && ldb % 16))
        return fail(H3Q_ERR_INVALID, "%s: lda/ldb must be multiples of 16 bytes", who);
    if (!aligned(a, 16) || !aligned(b, 16)) return fail(H3Q_ERR_INVALID, "%s: a/b must be 16-byte aligned", who);
    // Block-relative buffer offsets are 32-bit: 256 rows of the larger stride must stay below 2^31.
    if ((!a_tiled && lda >= (int64_t(1) << 23)) || (!b_tiled && ldb >= (int64_t(1) << 23)))
        return fail(H3Q_ERR_UNSUPPORTED, "%s: row stride above 8 MiB", who);
    if ((m + 255) / 256 * ((n + 255) / 256) >= (int64_t(1) << 31))
        return fail(H3Q_ERR_UNSUPPORTED, "%s: too many output tiles", who);
    // A 256-row tile of a tiled operand spans 256 * k bytes behind a 32-bit offset.
    if ((a_tiled || b_tiled) && 256 * k >= (int64_t(1) << 31))
        return fail(H3Q_ERR_UNSUPPORTED, "%s: tiled operands need 256 * k below 2^31", who);
    return H3Q_OK;
}

__attribute__((visibility("default"))) int h3q_scaled_mm(int format, const void* a, int64_t lda, int a_layout,
                                                         const float* a_scale, int a_scale_kind, const void* b,
                                                         int64_t ldb, int b_layout, const float* b_scale,
                                                         int b_scale_kind, const void* bias, const void* lora_t,
                                                         int64_t ldt, const void* lora_b, int64_t ldlb,
                                                         int64_t lora_rank, float lora_scale, void* out,
                                                         int64_t ldo, int64_t m, int64_t n, int64_t k, void* stream) {
    const char* who = "h3q_scaled_mm";
    const bool out_f16 = (format & H3Q_OUT_F16) != 0;
    format &= ~H3Q_OUT_F16;
    if (format != H3Q_FMT_E4M3FN && format != H3Q_FMT_INT8)
        return fail(H3Q_ERR_INVALID, "%s: unknown format %d", who, format);
    for (int layout : {a_layout, b_layout})
        if (layout != H3Q_LAYOUT_ROWS && layout != H3Q_LAYOUT_TILED)
            return fail(H3Q_ERR_INVALID, "%s: unknown operand layout %d", who, layout);
    const bool a_tiled = a_layout == H3Q_LAYOUT_TILED, b_tiled = b_layout == H3Q_LAYOUT_TILED;
    if (int rc = check_gemm_operands(who, a, lda, b, ldb, m, n, k, 1, a_tiled, b_tiled)) return rc;
    if (a_tiled && lora_t && m <= h3q::kSkinnyMaxM)
        return fail(H3Q_ERR_UNSUPPORTED, "%s: tiled activations with m <= %lld take no LoRA epilogue", who,
                    (long long)h3q::kSkinnyMaxM);
    for (int kind : {a_scale_kind, b_scale_kind})
        if (kind != H3Q_SCALE_PER_ROW && kind != H3Q_SCALE_PER_TENSOR)
            return fail(H3Q_ERR_INVALID, "%s: unknown scale kind %d", who, kind);
    if (ldo < n) return fail(H3Q_ERR_INVALID, "%s: ldo below n", who);
    // Block-relative output offsets are 32-bit: 256 rows of ldo 4-byte elements stay below 2^31.
    if (ldo >= (int64_t(1) << 21)) return fail(H3Q_ERR_UNSUPPORTED, "%s: output row stride above 2^21", who);
    if ((lora_t == nullptr) != (lora_b == nullptr))
        return fail(H3Q_ERR_INVALID, "%s: lora_t and lora_b must be given together", who);
    if (lora_t) {
        if (out_f16) return fail(H3Q_ERR_UNSUPPORTED, "%s: the LoRA epilogue writes bf16 only", who);
        if (lora_rank <= 0 || lora_rank > 128 || lora_rank % 8)
            return fail(H3Q_ERR_UNSUPPORTED, "%s: LoRA rank %lld (fused epilogue takes 8..128, multiple of 8)",
                        who, (long long)lora_rank);
        if (ldt < lora_rank || ldlb < lora_rank || ldt % 8 || ldlb % 8 || !aligned(lora_t, 16) ||
            !aligned(lora_b, 16))
            return fail(H3Q_ERR_INVALID, "%s: LoRA operands must be 16-byte aligned rows of >= rank", who);
        // 256 rows of either LoRA operand sit behind a 32-bit buffer offset.
        if (ldt * 2 >= (int64_t(1) << 23) || ldlb * 2 >= (int64_t(1) << 23))
            return fail(H3Q_ERR_UNSUPPORTED, "%s: LoRA row stride above 8 MiB", who);
    }
    // Tiled activations beyond the weight-streaming GEMM's rows are read by the
    // four-wave GEMM only (see w4_supported).
    if (a_tiled && m > h3q::kSkinnyMaxM && (k < 256 || n % 8 || ldo % 8 || !aligned(out, 16) || out_f16))
        return fail(H3Q_ERR_UNSUPPORTED,
                    "%s: tiled activations with m > %lld need k >= 256, n and ldo multiples of 8, a 16-byte "
                    "aligned output and bf16 output",
                    who, (long long)h3q::kSkinnyMaxM);
    if (m == 0 || n == 0) return ok();
    if (!a || !b || !a_scale || !b_scale || !out) return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    h3q::GemmArgs g{};
    g.a = a;
    g.b = b;
    g.lda = lda;
    g.ldb = ldb;
    g.m = m;
    g.n = n;
    g.k = k;
    g.a_scale = a_scale;
    g.b_scale = b_scale;
    g.a_scale_per_row = a_scale_kind == H3Q_SCALE_PER_ROW;
    g.b_scale_per_col = b_scale_kind == H3Q_SCALE_PER_ROW;
    g.bias = (const uint16_t*)bias;
    g.lora_t = (const uint16_t*)lora_t;
    g.lora_b = (const uint16_t*)lora_b;
    g.ldt = ldt;
    g.ldlb = ldlb;
    g.lora_rank = lora_rank;
    g.lora_scale = lora_scale;
    g.out = out;
    g.ldo = ldo;
    g.a_tiled = a_tiled;
    g.b_tiled = b_tiled;
    g.out_f16 = out_f16;
    const int kind = format == H3Q_FMT_E4M3FN ? h3q::kOpE4M3 : h3q::kOpInt8;
    return check_launch(h3q::launch_gemm(kind, false, g, (hipStream_t)stream), who);
}

__attribute__((visibility("default"))) int h3q_gemm_i8_i32(const void* a, int64_t lda, const void* b, int64_t ldb,
                                                           void* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                                                           void* stream) {
    const char* who = "h3q_gemm_i8_i32";
    if (int rc = check_gemm_operands(who, a, lda, b, ldb, m, n, k, 1)) return rc;
    if (ldo < n) return fail(H3Q_ERR_INVALID, "%s: ldo below n", who);
    // Block-relative output offsets are 32-bit: 256 rows of ldo 4-byte elements stay below 2^31.
    if (ldo >= (int64_t(1) << 21)) return fail(H3Q_ERR_UNSUPPORTED, "%s: output row stride above 2^21", who);
    if (m == 0 || n == 0) return ok();
    if (!a || !b || !out) return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    h3q::GemmArgs g{};
    g.a = a;
    g.b = b;
    g.lda = lda;
    g.ldb = ldb;
    g.m = m;
    g.n = n;
    g.k = k;
    g.out = out;
    g.ldo = ldo;
    return check_launch(h3q::launch_gemm(h3q::kOpInt8, true, g, (hipStream_t)stream), who);
}

static int lora_down_args(const char* who, const void* x, int64_t ldx, const void* lora_a, int64_t lda, void* t,
                          int64_t ldt, int64_t m, int64_t k, int64_t rank, h3q::GemmArgs& g) {
    if (k % 8) return fail(H3Q_ERR_INVALID, "%s: k=%lld must be a multiple of 8", who, (long long)k);
    if (m < 0 || k < 0 || rank <= 0) return fail(H3Q_ERR_INVALID, "%s: bad shape", who);
    if (ldx < k || lda < k || ldt < rank) return fail(H3Q_ERR_INVALID, "%s: leading dimension too small", who);
    if (ldt >= (int64_t(1) << 21)) return fail(H3Q_ERR_UNSUPPORTED, "%s: output row stride above 2^21", who);
    if (ldx % 8 || lda % 8 || !aligned(x, 16) || !aligned(lora_a, 16))
        return fail(H3Q_ERR_INVALID, "%s: x / lora_a rows must be 16-byte aligned", who);
    if (ldx * 2 >= (int64_t(1) << 23) || lda * 2 >= (int64_t(1) << 23))
        return fail(H3Q_ERR_UNSUPPORTED, "%s: row stride above 8 MiB", who);
    if (m == 0) return H3Q_OK;
    if (!x || !lora_a || !t) return fail(H3Q_ERR_INVALID, "%s: null pointer", who);
    g = h3q::GemmArgs{};
    g.a = x;
    g.b = lora_a;
    g.lda = ldx * 2;
    g.ldb = lda * 2;
    g.m = m;
    g.n = rank;
    g.k = k;
    g.out = t;
    g.ldo = ldt;
    return H3Q_OK;
}

__attribute__((visibility("default"))) int h3q_lora_down(const void* x, int64_t ldx, const void* lora_a,
                                                         int64_t lda, void* t, int64_t ldt, int64_t m, int64_t k,
                                                         int64_t rank, void* stream) {
    const char* who = "h3q_lora_down";
    h3q::GemmArgs g{};
    const int rc = lora_down_args(who, x, ldx, lora_a, lda, t, ldt, m, k, rank, g);
    if (rc != H3Q_OK || m == 0) return rc == H3Q_OK ? ok() : rc;
    return check_launch(h3q::launch_gemm(h3q::kOpBF16, false, g, (hipStream_t)stream), who);
}

__attribute__((visibility("default"))) int64_t h3q_lora_down_workspace_bytes(int64_t m, int64_t k, int64_t rank) {
    if (m <= 0 || k <= 0 || rank <= 0) return 0;
    return h3q::lora_down_workspace_bytes(m, k, rank);
}

__attribute__((visibility("default"))) int h3q_lora_down_ws(const void* x, int64_t ldx, const void* lora_a,
                                                            int64_t lda, void* t, int64_t ldt, int64_t m, int64_t k,
                                                            int64_t rank, void* workspace, int64_t workspace_bytes,
                                                            void* stream) {
    const char* who = "h3q_lora_down_ws";
    h3q::GemmArgs g{};
    const int rc = lora_down_args(who, x, ldx, lora_a, lda, t, ldt, m, k, rank, g);
    if (rc != H3Q_OK || m == 0) return rc == H3Q_OK ? ok() : rc;
    const int64_t need = h3q::lora_down_workspace_bytes(m, k, rank);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(H3Q_ERR_INVALID, "%s: workspace of %lld bytes needed, %lld given", who, (long long)need,
                    (long long)workspace_bytes);
    if (need > 0 && !aligned(workspace, 16)) return fail(H3Q_ERR_INVALID, "%s: workspace must be 16-byte aligned", who);
    return check_launch(h3q::launch_lora_down(g, workspace, workspace_bytes, (hipStream_t)stream), who);
}

}  // extern "C"
