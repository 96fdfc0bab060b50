// act.hpp -- bias / activation selectors and the activation functions shared
// by the int8-out and fp8-out GEMM epilogues
// (baracuda_epilogue_int8.cuh:37-84 semantics: relu, exact-erf gelu, silu).
#pragma once

#include "bk_common.hpp"

namespace bk {
namespace {

enum Act : int { ACT_NONE = 0, ACT_BIAS = 1, ACT_BIAS_RELU = 2, ACT_BIAS_GELU = 3, ACT_BIAS_SILU = 4 };

// exp(x) through the hardware base-2 exponential (v_exp_f32, 1 ulp).
__device__ __forceinline__ float exp_hw(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f);
}

// erf(x) by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7): branch-free, one
// reciprocal and one exponential, against ~40 instructions with branches for
// libm erff.  One 256x256 tile per CU makes the epilogue 128 activations per
// thread, so this is what keeps the Gelu SKU close to the Identity one.
__device__ __forceinline__ float erf_as7126(float x) {
    const float ax = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, ax, 1.0f));
    float poly = fmaf(1.061405429f, t, -1.453152027f);
    poly = fmaf(poly, t, 1.421413741f);
    poly = fmaf(poly, t, -0.284496736f);
    poly = fmaf(poly, t, 0.254829592f);
    const float y = 1.0f - poly * t * exp_hw(-ax * ax);
    return copysignf(y, x);
}

template <int ACT>
__device__ __forceinline__ float activation(float x) {
    if constexpr (ACT == ACT_BIAS_RELU) return fmaxf(x, 0.0f);
    else if constexpr (ACT == ACT_BIAS_GELU) return 0.5f * x * (1.0f + erf_as7126(x * 0.70710678118654752440f));
    else if constexpr (ACT == ACT_BIAS_SILU) return x * __builtin_amdgcn_rcpf(1.0f + exp_hw(-x));
    else return x;
}

}  // namespace
}  // namespace bk
