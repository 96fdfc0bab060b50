// gemm_fp8_bias.hip -- e4m3 RCR / RRR GEMM with the bias / activation
// epilogue family: D = sat_e4m3(act(alpha*acc + beta*dequant(C) + bias[n])),
// bias f32 [N].  Same ABI as baracuda_kernels_gemm_fp8_e4m3_{rcr,rrr}_sm89_{bias,
// bias_relu,bias_gelu,bias_silu}_* (kernels/gemm/gemm_fp8_e4m3_{rcr,rrr}_sm89_bias.cu).
#include "gemm_fp8_kernels.hpp"

using namespace bk;

extern "C" {
BK_FP8_BIAS_FAMILY(e4m3, rcr, FMT_E4M3, F8_RCR)
BK_FP8_BIAS_FAMILY(e4m3, rrr, FMT_E4M3, F8_RRR)
}  // extern "C"
