// gemm_fp8.hip -- FP8 GEMM SKUs for gfx950: e4m3 RCR / RRR with the
// reference's fp8-out epilogue, the e4m3 RCR bf16 / f32-out SKUs, and e5m2
// RCR / RRR.
//
// Replaces baracuda_kernels_gemm_fp8_{e4m3,e5m2}_{rcr,rrr}_sm89_*
// (crates/baracuda-kernels-sys/kernels/gemm/gemm_fp8_{e4m3,e5m2}_{rcr,rrr}_sm89.cu):
//   (plain)  D = sat_fp8(alpha*acc + beta*dequant(C))       reference semantics
//   _bf16    D = bf16_rne((scale_a*scale_b) * acc)          new SKU (per-tensor scales)
//   _f32     D = alpha * acc                                 new SKU (accumulator check)
#include "gemm_fp8_kernels.hpp"

using namespace bk;

extern "C" {

BK_FP8_IDENTITY_SKU(e4m3, rcr, FMT_E4M3, F8_RCR)
BK_FP8_IDENTITY_SKU(e4m3, rrr, FMT_E4M3, F8_RRR)
BK_FP8_IDENTITY_SKU(e5m2, rcr, FMT_E5M2, F8_RCR)
BK_FP8_IDENTITY_SKU(e5m2, rrr, FMT_E5M2, F8_RRR)

// ---- bf16 out with per-tensor scales (new SKU) ------------------------------
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return check_fp8<F8_RCR>(m, n, k, lda, ldb, nullptr, 0, ldd);
}

size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    float scale_a, float scale_b, void *d, int64_t ldd,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = check_fp8<F8_RCR>(m, n, k, lda, ldb, nullptr, 0, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    F8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd,
             scale_a * scale_b, 0.0f, nullptr};
    return launch_fp8<FMT_E4M3, F8_RCR, F8_BF16, ACT_NONE>(p, (hipStream_t)stream);
}

// ---- f32 out: D = alpha * acc (new SKU, exposes the accumulator) ------------
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return check_fp8<F8_RCR>(m, n, k, lda, ldb, nullptr, 0, ldd);
}

size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    float alpha, void *d, int64_t ldd, void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = check_fp8<F8_RCR>(m, n, k, lda, ldb, nullptr, 0, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    F8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd, alpha, 0.0f,
             nullptr};
    return launch_fp8<FMT_E4M3, F8_RCR, F8_F32, ACT_NONE>(p, (hipStream_t)stream);
}

}  // extern "C"
