// gemm_s8_bias.hip -- int8 RCR GEMM with the bias / activation epilogue
// family for gfx950 (same kernels as gemm_s8.hip, bias/act instantiations).
#include "gemm_s8_kernels.hpp"

using namespace bk;

namespace {
int32_t bk_rcr_can(int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b,
                   int64_t ldb, const void *c, int64_t ldc, void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (c != nullptr && ldc < n) return kInvalid;
    return kOk;
}
}  // namespace

extern "C" {

// ---- int8 RCR with bias / activation epilogue -------------------------------
// Same ABI as baracuda_kernels_gemm_{bias,bias_relu,bias_gelu,bias_silu}_{f32bias,i32bias}_s8_rcr_sm80_*
// (crates/baracuda-cutlass-kernels-sys/kernels/gemm_s8_rcr_sm80_bias.cu:225-275,
//  re-exported in crates/baracuda-kernels-sys/src/cutlass_reexport.rs:1025-).
// D = sat_s8(rne(act(alpha*acc + beta*C + bias[n]))).
#define BK_S8_RCR_BIAS(EPISFX, ACTV, BSFX, BTY)                                                      \
    int32_t baracuda_kernels_gemm_##EPISFX##_##BSFX##_s8_rcr_gfx950_can_implement(                  \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,     \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias) {                        \
        int32_t st = bk_rcr_can(m, n, k, a, lda, b, ldb, c,   \
                                                                      ldc, d, ldd);                  \
        if (st != kOk) return st;                                                                    \
        (void)bias;                                                                                  \
        return kOk;                                                                                  \
    }                                                                                                \
    size_t baracuda_kernels_gemm_##EPISFX##_##BSFX##_s8_rcr_gfx950_workspace_size(int32_t m,         \
                                                                                int32_t n, int32_t k) { \
        return tail_split_workspace(m, n, k);                                                        \
    }                                                                                                \
    int32_t baracuda_kernels_gemm_##EPISFX##_##BSFX##_s8_rcr_gfx950_run(                            \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,     \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha, float beta, \
        void *workspace, size_t workspace_bytes, void *stream) {                                     \
        int32_t st = bk_rcr_can(m, n, k, a, lda, b, ldb, c,   \
                                                                      ldc, d, ldd);                  \
        if (st != kOk) return st;                                                                    \
        if (!a || !b || !d || !bias) return kInvalid;                                                \
        S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, \
                 ldd, alpha, beta, nullptr, nullptr, bias};                                          \
        rcr_c_defaults_to_d(p);                                                                      \
        return launch<EPI_S8, ACTV, BTY>(p, (hipStream_t)stream, workspace, workspace_bytes);        \
    }

BK_S8_RCR_BIAS(bias, ACT_BIAS, f32bias, float)
BK_S8_RCR_BIAS(bias_relu, ACT_BIAS_RELU, f32bias, float)
BK_S8_RCR_BIAS(bias_gelu, ACT_BIAS_GELU, f32bias, float)
BK_S8_RCR_BIAS(bias_silu, ACT_BIAS_SILU, f32bias, float)
BK_S8_RCR_BIAS(bias, ACT_BIAS, i32bias, int32_t)
BK_S8_RCR_BIAS(bias_relu, ACT_BIAS_RELU, i32bias, int32_t)
BK_S8_RCR_BIAS(bias_gelu, ACT_BIAS_GELU, i32bias, int32_t)
BK_S8_RCR_BIAS(bias_silu, ACT_BIAS_SILU, i32bias, int32_t)
#undef BK_S8_RCR_BIAS

}  // extern "C"
