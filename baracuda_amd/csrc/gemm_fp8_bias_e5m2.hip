// gemm_fp8_bias_e5m2.hip -- e5m2 RCR / RRR GEMM with the bias / activation
// epilogue family: D = sat_e5m2(act(alpha*acc + beta*dequant(C) + bias[n])),
// bias f32 [N].  Same ABI as baracuda_kernels_gemm_fp8_e5m2_{rcr,rrr}_sm89_{bias,
// bias_relu,bias_gelu,bias_silu}_* (kernels/gemm/gemm_fp8_e5m2_{rcr,rrr}_sm89_bias.cu).
#include "gemm_fp8_kernels.hpp"

using namespace bk;

extern "C" {
BK_FP8_BIAS_FAMILY(e5m2, rcr, FMT_E5M2, F8_RCR)
BK_FP8_BIAS_FAMILY(e5m2, rrr, FMT_E5M2, F8_RRR)
}  // extern "C"
