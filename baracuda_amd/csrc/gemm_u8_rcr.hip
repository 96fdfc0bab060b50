// gemm_u8_rcr.hip -- u8 x u8 RCR GEMM (B [N, K], the "column-major [K, N]"
// operand) and its bias / activation family for gfx950:
// D = sat_u8(rne(act(alpha*acc + beta*C [+ bias[n]]))), acc the exact int32
// sum of u8 products, C and D u8.
//
// gfx950's int8 MFMA is signed, so operands run through it as u - 128 and the
// kernels add the row / column-sum correction back (gemm_s8_kernels.hpp).
#include "gemm_s8_kernels.hpp"

using namespace bk;

namespace {
int32_t u8_rcr_can(int32_t m, int32_t n, int32_t k, int64_t lda, int64_t ldb, const void *c, int64_t ldc,
                   int64_t ldd) {
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (c != nullptr && ldc < n) return kInvalid;
    return kOk;
}
}  // namespace

extern "C" {

// Same ABI as baracuda_kernels_gemm_u8_rcr_sm80_{run,workspace_size,can_implement}
// (crates/baracuda-cutlass-kernels-sys/kernels/gemm_u8_rcr_sm80.cu, re-exported at
//  crates/baracuda-kernels-sys/src/cutlass_reexport.rs:669-676).  No workspace.
int32_t baracuda_kernels_gemm_u8_rcr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return u8_rcr_can(m, n, k, lda, ldb, c, ldc, ldd);
}

size_t baracuda_kernels_gemm_u8_rcr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_u8_rcr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = u8_rcr_can(m, n, k, lda, ldb, c, ldc, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, ldd,
             alpha, beta, nullptr, nullptr, nullptr};
    rcr_c_defaults_to_d(p);
    return launch_u8_rcr<ACT_NONE, float>(p, (hipStream_t)stream);
}

// Same ABI as baracuda_kernels_gemm_{bias,bias_relu,bias_gelu,bias_silu}_{f32bias,i32bias}_u8_rcr_sm80_*
// (crates/baracuda-cutlass-kernels-sys/kernels/gemm_u8_rcr_sm80_bias.cu, re-exported at
//  crates/baracuda-kernels-sys/src/cutlass_reexport.rs:1062-1096 (f32bias) and 1141-1176 (i32bias)).
#define BK_U8_RCR_BIAS(EPISFX, ACTV, BSFX, BTY)                                                      \
    int32_t baracuda_kernels_gemm_##EPISFX##_##BSFX##_u8_rcr_gfx950_can_implement(                  \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,     \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias) {                        \
        (void)a; (void)b; (void)d; (void)bias;                                                       \
        return u8_rcr_can(m, n, k, lda, ldb, c, ldc, ldd);                                           \
    }                                                                                                \
    size_t baracuda_kernels_gemm_##EPISFX##_##BSFX##_u8_rcr_gfx950_workspace_size(int32_t m,         \
                                                                                int32_t n, int32_t k) { \
        (void)m; (void)n; (void)k;                                                                   \
        return 0;                                                                                    \
    }                                                                                                \
    int32_t baracuda_kernels_gemm_##EPISFX##_##BSFX##_u8_rcr_gfx950_run(                            \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,     \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha, float beta, \
        void *workspace, size_t workspace_bytes, void *stream) {                                     \
        (void)workspace; (void)workspace_bytes;                                                      \
        int32_t st = u8_rcr_can(m, n, k, lda, ldb, c, ldc, ldd);                                     \
        if (st != kOk) return st;                                                                    \
        if (!a || !b || !d || !bias) return kInvalid;                                                \
        S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, \
                 ldd, alpha, beta, nullptr, nullptr, bias};                                          \
        rcr_c_defaults_to_d(p);                                                                      \
        return launch_u8_rcr<ACTV, BTY>(p, (hipStream_t)stream);                                     \
    }

BK_U8_RCR_BIAS(bias, ACT_BIAS, f32bias, float)
BK_U8_RCR_BIAS(bias_relu, ACT_BIAS_RELU, f32bias, float)
BK_U8_RCR_BIAS(bias_gelu, ACT_BIAS_GELU, f32bias, float)
BK_U8_RCR_BIAS(bias_silu, ACT_BIAS_SILU, f32bias, float)
BK_U8_RCR_BIAS(bias, ACT_BIAS, i32bias, int32_t)
BK_U8_RCR_BIAS(bias_relu, ACT_BIAS_RELU, i32bias, int32_t)
BK_U8_RCR_BIAS(bias_gelu, ACT_BIAS_GELU, i32bias, int32_t)
BK_U8_RCR_BIAS(bias_silu, ACT_BIAS_SILU, i32bias, int32_t)
#undef BK_U8_RCR_BIAS

}  // extern "C"
