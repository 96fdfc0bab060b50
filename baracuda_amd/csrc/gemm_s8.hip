// gemm_s8.hip -- int8 RCR GEMM SKUs for gfx950 (v_mfma_i32_16x16x64_i8).
//
// Replaces the CUTLASS int8 RCR GEMM
// (crates/baracuda-cutlass-kernels-sys/kernels/gemm_s8_rcr_sm80.cu:41-198)
// and the naive W8A8 quantized-linear kernel
// (crates/baracuda-kernels-sys/kernels/include/baracuda_quantize_compose.cuh:246-372)
// with one MFMA mainloop and four epilogues:
//   _i32      D = acc (int32)                                  new SKU
//   (plain)   D = sat_s8(rne(alpha*acc + beta*C))              gemm_s8_rcr_sm80 semantics
//   w8a8 bf16 D = bf16_rne((sa[m]*sw[n]) * (float)acc)          new SKU
//   w8a8 f32  D = (sa[m]*sw[n]) * (float)acc                    quantized_linear_w8a8_f32
//   w8a8 f64  D = (double)(((float)sa[m]*(float)sw[n]) * (float)acc)  quantized_linear_w8a8_f64
//
// The accumulator wraps modulo 2^32 where the reference's mma.sync
// saturates; the two agree whenever |acc| < 2^31, which holds for int8
// operands in [-127,127] whenever K < 133143.
#include "gemm_s8_kernels.hpp"

using namespace bk;

extern "C" {

// ---- int8 RCR, int32 output (new SKU) -------------------------------------
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return check_rcr(m, n, k, lda, ldb, ldd);
}

size_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_workspace_size(int32_t m, int32_t n, int32_t k) {
    return tail_split_workspace(m, n, k);
}

int32_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    void *d, int64_t ldd, void *workspace, size_t workspace_bytes, void *stream) {
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd,
             1.0f, 0.0f, nullptr, nullptr, nullptr};
    return launch<EPI_I32>(p, (hipStream_t)stream, workspace, workspace_bytes);
}

// ---- int8 RCR, int8 output: D = sat_s8(alpha*acc + beta*C) ------------------
// Same ABI as baracuda_kernels_gemm_s8_rcr_sm80_* (gemm_s8_rcr_sm80.cu:169-198).
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (c != nullptr && ldc < n) return kInvalid;
    return kOk;
}

size_t baracuda_kernels_gemm_s8_rcr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k) {
    return tail_split_workspace(m, n, k);
}

int32_t baracuda_kernels_gemm_s8_rcr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream) {
    int32_t st = baracuda_kernels_gemm_s8_rcr_gfx950_can_implement(m, n, k, a, lda, b, ldb, c, ldc, d, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, ldd,
             alpha, beta, nullptr, nullptr, nullptr};
    rcr_c_defaults_to_d(p);
    return launch<EPI_S8>(p, (hipStream_t)stream, workspace, workspace_bytes);
}

// ---- W8A8: D = bf16((scale_a[m] * scale_b[n]) * acc) (new SKU) -----------
int32_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *scale_a, const void *scale_b, const void *d, int64_t ldd) {
    (void)a; (void)b; (void)scale_a; (void)scale_b; (void)d;
    return check_rcr(m, n, k, lda, ldb, ldd);
}

size_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_workspace_size(int32_t m, int32_t n, int32_t k) {
    return tail_split_workspace(m, n, k);
}

int32_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const float *scale_a, const float *scale_b, void *d, int64_t ldd,
    void *workspace, size_t workspace_bytes, void *stream) {
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d || !scale_a || !scale_b) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd,
             1.0f, 0.0f, scale_a, scale_b, nullptr};
    return launch<EPI_W8A8_BF16>(p, (hipStream_t)stream, workspace, workspace_bytes);
}

// ---- quantized_linear_w8a8 f32 (baracuda_quantize_compose.cuh:340-370 ABI) --
// y[m, c] = scale_a[m] * scale_w[c] * acc, weight [C_out, K], act [M, K].
int32_t baracuda_kernels_quantized_linear_w8a8_f32_gfx950_can_implement(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, const void *output) {
    (void)weight_q; (void)act_q; (void)scale_a; (void)scale_w; (void)output;
    if (M < 0 || C_out < 0 || K < 0) return kInvalid;
    return kOk;
}

int32_t baracuda_kernels_quantized_linear_w8a8_f32_gfx950_run(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, void *output,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    if (M < 0 || C_out < 0 || K < 0) return kInvalid;
    if ((int64_t)M * C_out == 0) return kOk;
    if (!weight_q || !act_q || !scale_a || !scale_w || !output) return kInvalid;
    if (K == 0) {
        // Empty reduction: acc = 0 for every cell, handled by a K=0 tile pass.
        S8Args p{M, C_out, 0, (const int8_t *)act_q, 0, (const int8_t *)weight_q, 0, nullptr, 0,
                 output, C_out, 1.0f, 0.0f, (const float *)scale_a, (const float *)scale_w, nullptr};
        return launch<EPI_W8A8_F32>(p, (hipStream_t)stream);
    }
    S8Args p{M, C_out, K, (const int8_t *)act_q, K, (const int8_t *)weight_q, K, nullptr, 0,
             output, C_out, 1.0f, 0.0f, (const float *)scale_a, (const float *)scale_w, nullptr};
    return launch<EPI_W8A8_F32>(p, (hipStream_t)stream);
}

// ---- quantized_linear_w8a8 f64 (compose.cu:27-28, same ABI) ----------------
// f64 scales and output; the reference kernel narrows the scales to f32
// (qc_load_as_f32), forms y = sa*sw*(float)acc in f32 and widens y to f64
// (baracuda_quantize_compose.cuh:265-274, qc_store_from_f32<double>).
int32_t baracuda_kernels_quantized_linear_w8a8_f64_gfx950_can_implement(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, const void *output) {
    (void)weight_q; (void)act_q; (void)scale_a; (void)scale_w; (void)output;
    if (M < 0 || C_out < 0 || K < 0) return kInvalid;
    return kOk;
}

int32_t baracuda_kernels_quantized_linear_w8a8_f64_gfx950_run(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, void *output,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    if (M < 0 || C_out < 0 || K < 0) return kInvalid;
    if ((int64_t)M * C_out == 0) return kOk;
    if (!weight_q || !act_q || !scale_a || !scale_w || !output) return kInvalid;
    // The scale pointers travel in S8Args' f32 slots and are read as f64 by
    // the EPI_W8A8_F64 epilogue; K == 0 runs the same tile pass with acc = 0.
    S8Args p{M, C_out, K, (const int8_t *)act_q, K, (const int8_t *)weight_q, K, nullptr, 0,
             output, C_out, 1.0f, 0.0f, (const float *)scale_a, (const float *)scale_w, nullptr};
    return launch<EPI_W8A8_F64>(p, (hipStream_t)stream);
}

}  // extern "C"
