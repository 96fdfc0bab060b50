// bk_common.hpp -- shared vocabulary of the gfx950 kernels behind the
// baracuda_kernels_* C ABI: status codes, vector types and the exact scalar
// codecs (bf16 RNE, OCP e4m3) the epilogues use.
//
// Status codes are the reference's (crates/baracuda-kernels-sys/src/lib.rs:19-27):
//   0 ok, 1 misaligned, 2 invalid problem, 3 unsupported, 4 workspace, 5 launch.
#pragma once

#include <hip/hip_runtime.h>

#include "baracuda_kernels.h"
#include <cstddef>
#include <cstdint>

namespace bk {

enum Status : int32_t {
    kOk = 0,
    kMisaligned = 1,
    kInvalid = 2,
    kUnsupported = 3,
    kWorkspace = 4,
    kLaunch = 5,
};

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

inline int32_t launch_status() {
    return hipPeekAtLastError() == hipSuccess ? kOk : kLaunch;
}

// f32 -> bf16 bits, round to nearest even; NaN keeps its top half with the
// quiet bit set (crates/baracuda-kernelgen/src/oracle.rs:397-404).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    uint32_t bits = __float_as_uint(x);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t bias = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + bias) >> 16);
}

// Two f32 -> packed bf16x2 (low half = lo) with the gfx950 conversion
// instruction v_cvt_pk_bf16_f32: round to nearest even, so finite values
// round exactly like f32_to_bf16_rne (a NaN stays a quiet NaN, payload not
// guaranteed).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

// f32 -> f16 bits, round to nearest even, overflow to inf, NaN quiet.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float x) {
    _Float16 h = (_Float16)x;   // v_cvt_f16_f32 rounds to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// OCP E4M3 (e4m3fn) saturating encode with round-to-nearest-even, written
// from the format definition: bias 7, max finite 448 (S.1111.110), NaN
// S.1111.111, subnormals m * 2^-9.  |x| > 448 (and +-inf) clamps to +-448.
__device__ __forceinline__ uint8_t f32_to_e4m3_satfinite(float x) {
    uint32_t bits = __float_as_uint(x);
    uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
    uint32_t abs = bits & 0x7fffffffu;
    if (abs > 0x7f800000u) return (uint8_t)(sign | 0x7f);
    if (abs >= 0x43e00000u) return (uint8_t)(sign | 0x7e);   // >= 448 (incl. inf)
    if (abs < 0x3c800000u) {                                  // < 2^-6: subnormal grid
        float q = __builtin_rintf(__uint_as_float(abs) * 512.0f);
        return (uint8_t)(sign | (uint8_t)q);                  // q == 8 -> min normal
    }
    // Normal: keep 3 mantissa bits with RNE on the f32 bit pattern.
    uint32_t lsb = (abs >> 20) & 1u;
    uint32_t r = abs + 0x7ffffu + lsb;
    uint32_t e = (r >> 23) - 127 + 7;
    uint32_t m = (r >> 20) & 7u;
    if (e > 15 || (e == 15 && m == 7)) return (uint8_t)(sign | 0x7e);
    return (uint8_t)(sign | (uint8_t)(e << 3) | (uint8_t)m);
}

__device__ __forceinline__ float e4m3_to_f32(uint8_t b) {
    uint32_t s = (uint32_t)(b & 0x80u) << 24;
    uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    if (e == 15 && m == 7) return __uint_as_float(s | 0x7fc00000u);
    if (e == 0) {
        float v = (float)m * (1.0f / 512.0f);
        return __uint_as_float(__float_as_uint(v) | s);
    }
    return __uint_as_float(s | ((e - 7 + 127) << 23) | (m << 20));
}

// OCP E5M2 saturating encode with round-to-nearest-even (the satfinite cast
// of baracuda_dtype.cuh:54-57): NaN stays NaN, |x| > 57344 (and inf) -> the
// max finite 0x7b, 2 mantissa bits kept with RNE on the f32 bit pattern,
// subnormals on the 2^-16 grid.
__device__ __forceinline__ uint8_t f32_to_e5m2_satfinite(float x) {
    uint32_t bits = __float_as_uint(x);
    uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
    uint32_t abs = bits & 0x7fffffffu;
    if (abs > 0x7f800000u) return (uint8_t)(sign | 0x7f);
    if (abs > 0x47600000u) return (uint8_t)(sign | 0x7b);   // > 57344 (incl. inf)
    if (abs < 0x38800000u) {                                  // < 2^-14: subnormal grid
        float q = __builtin_rintf(__uint_as_float(abs) * 65536.0f);
        return (uint8_t)(sign | (uint8_t)q);                  // q == 4 -> min normal
    }
    uint32_t lsb = (abs >> 21) & 1u;
    uint32_t r = abs + 0xfffffu + lsb;
    uint32_t e = (r >> 23) - 127 + 15;
    uint32_t m = (r >> 21) & 3u;
    if (e > 30) return (uint8_t)(sign | 0x7b);
    return (uint8_t)(sign | (uint8_t)(e << 2) | (uint8_t)m);
}

// E5M2 is the top byte of an IEEE binary16.
__device__ __forceinline__ float e5m2_to_f32(uint8_t b) { return f16_to_f32((uint16_t)((uint16_t)b << 8)); }

// fp8 format selector shared by the kernels and the MFMA cbsz / blgp fields.
enum Fp8Fmt : int { FMT_E4M3 = 0, FMT_E5M2 = 1 };

// fp8 byte -> f32 through the hardware conversion (v_cvt_f32_fp8 /
// v_cvt_f32_bf8: the OCP formats on gfx950; exact for every non-NaN code,
// tested against e4m3_to_f32 / e5m2_to_f32 over all 256 codes).  NaN codes
// give a quiet NaN carrying the code's sign, as the software decoders do
// (the encoders below map a NaN to sign | 0x7f).
template <int FMT>
__device__ __forceinline__ float fp8_to_f32(uint8_t b) {
    const float v = FMT == FMT_E5M2 ? __builtin_amdgcn_cvt_f32_bf8((int)b, 0)
                                    : __builtin_amdgcn_cvt_f32_fp8((int)b, 0);
    const bool nan = FMT == FMT_E5M2 ? (b & 0x7fu) > 0x7cu : (b & 0x7fu) == 0x7fu;
    return nan ? __uint_as_float(((uint32_t)(b & 0x80u) << 24) | 0x7fc00000u) : v;
}

template <int FMT>
__device__ __forceinline__ uint8_t f32_to_fp8_satfinite(float x) {
    if constexpr (FMT == FMT_E5M2) return f32_to_e5m2_satfinite(x);
    else return f32_to_e4m3_satfinite(x);
}

// Four f32 -> four satfinite fp8 bytes (byte i = element i) through the
// hardware packed conversion (v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32, RNE).
// Measured on gfx950 to equal f32_to_fp8_satfinite bit for bit for every
// |x| <= max finite (2^24 patterns spanning all exponents, ties and
// subnormals); beyond that the instruction overflows to NaN / inf and gives
// NaN the sign bit, so the input is clamped to +-max first and NaN inputs
// take the software code (sign | 0x7f).
template <int FMT>
__device__ __forceinline__ uint32_t f32x4_to_fp8x4_satfinite(float a, float b, float c, float d) {
    constexpr float M = FMT == FMT_E5M2 ? 57344.0f : 448.0f;
    const float ca = fminf(fmaxf(a, -M), M), cb = fminf(fmaxf(b, -M), M);
    const float cc = fminf(fmaxf(c, -M), M), cd = fminf(fmaxf(d, -M), M);
    uint32_t w;
    if constexpr (FMT == FMT_E5M2) {
        w = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(ca, cb, 0, false);
        w = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(cc, cd, (int)w, true);
    } else {
        w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false);
        w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(cc, cd, (int)w, true);
    }
    const float v[4] = {a, b, c, d};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (v[i] != v[i]) {
            const uint32_t nan = ((__float_as_uint(v[i]) >> 24) & 0x80u) | 0x7fu;
            w = (w & ~(0xffu << (8 * i))) | (nan << (8 * i));
        }
    }
    return w;
}

// 16-bit float MFMA operands: 8 elements = one 16-byte fragment word group.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// v_mfma_f32_16x16x32_{bf16,f16} on 16-byte fragments (srcA, srcB as raw words).
template <bool IsBf16>
__device__ __forceinline__ v4f mfma16x16x32_h(const v4i &a, const v4i &b, const v4f &c) {
    if constexpr (IsBf16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// u8 -> s8 operand flip for the signed int8 MFMA: each byte u becomes
// s = u - 128 (xor 0x80).
__device__ __forceinline__ v4i u8_flip(const v4i &f) {
    return v4i{f[0] ^ (int)0x80808080u, f[1] ^ (int)0x80808080u, f[2] ^ (int)0x80808080u,
               f[3] ^ (int)0x80808080u};
}

// Sum of the 16 raw bytes of a 16-byte chunk added to acc (v_dot4_u32_u8).
__device__ __forceinline__ uint32_t u8_sum16(const v4i &f, uint32_t acc) {
#pragma unroll
    for (int w = 0; w < 4; ++w) acc = __builtin_amdgcn_udot4((uint32_t)f[w], 0x01010101u, acc, false);
    return acc;
}


// Round half to even, clamp, convert (the reference's __float2int_rn + max /
// min, baracuda_dtype.cuh:23-36).  The clamp happens in float before the
// conversion, so the conversion is always of an in-range integral value and
// its result is defined by the language; NaN is mapped to 0 explicitly.
// rint, a NaN select, one v_med3_f32 and the conversion.
__device__ __forceinline__ float rne_clamp(float x, float lo, float hi) {
    float r = __builtin_rintf(x);
    r = (r == r) ? r : 0.0f;
    return __builtin_amdgcn_fmed3f(r, lo, hi);
}

__device__ __forceinline__ uint8_t sat_cast_u8(float x) {
    return (uint8_t)(int)rne_clamp(x, 0.0f, 255.0f);
}

__device__ __forceinline__ int8_t sat_cast_s8(float x) {
    return (int8_t)(int)rne_clamp(x, -128.0f, 127.0f);
}

}  // namespace bk
