/*
 * oracle.c -- CPU restatement of baracuda's reference arithmetic for the
 * quantized-inference contraction path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * The Rust originals (crates/baracuda-kernelgen/src/oracle.rs and the CPU
 * reference loops inside crates/baracuda-kernels/tests/ files) cannot be
 * compiled here (no rustc), so they are restated from the source text.
 * Citations are relative to the baracuda repository root.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* oracle.rs:397-404 f32_to_bf16_bits: NaN keeps its top half and sets the
 * quiet bit; otherwise add 0x7fff + lsb and truncate (RNE). */
uint16_t bo_f32_to_bf16_bits(float x) {
    uint32_t bits = f32_bits(x);
    if (isnan(x)) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t bias = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + bias) >> 16);
}

float bo_bf16_bits_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* oracle.rs f32_to_f16_bits (RNE, overflow -> inf, NaN quiet), restated as
 * exact arithmetic on the double value. */
uint16_t bo_f32_to_f16_bits(float x) {
    uint32_t bits = f32_bits(x);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    if (isnan(x)) return (uint16_t)(sign | 0x7e00u);
    double a = fabs((double)x);
    if (isinf(x) || a >= 65520.0) return (uint16_t)(sign | 0x7c00u);
    if (a < ldexp(1.0, -14)) {                 /* subnormal: units of 2^-24 */
        double q = nearbyint(a * ldexp(1.0, 24));
        return (uint16_t)(sign | (uint16_t)q);    /* q==1024 -> min normal */
    }
    int e;
    double m = frexp(a, &e);                   /* a = m*2^e, m in [0.5,1) */
    e -= 1; m *= 2.0;                          /* m in [1,2) */
    double q = nearbyint((m - 1.0) * 1024.0);
    if (q >= 1024.0) { q = 0.0; e += 1; }
    if (e + 15 >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)((e + 15) << 10) | (uint16_t)q);
}

float bo_f16_bits_to_f32(uint16_t h) {
    int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp(1.0 + m / 1024.0, e - 15);
    return (float)(s ? -v : v);
}

/* OCP 8-bit floating point spec, E4M3 ("E4M3FN"): bias 7, no infinities,
 * S.1111.111 is NaN, max finite 448 (S.1111.110), subnormals m/8 * 2^-6.
 * Replaces the crates.io `float8 0.7.0` codec used by
 * crates/baracuda-kernels/tests/fp8_e4m3_rcr_smoke.rs:27,36-43. */
float bo_e4m3_to_f32(uint8_t b) {
    int s = b >> 7, e = (b >> 3) & 0xf, m = b & 7;
    double v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexp((double)m, -9);
    else v = ldexp(1.0 + m / 8.0, e - 7);
    return (float)(s ? -v : v);
}

/* Saturating RNE encode to E4M3 (baracuda_dtype.cuh:39-46 semantics:
 * |x| beyond max-finite clamps to 448 instead of overflowing; NaN -> NaN). */
uint8_t bo_f32_to_e4m3_satfinite(float x) {
    uint8_t sign = (f32_bits(x) >> 24) & 0x80u;
    if (isnan(x)) return (uint8_t)(sign | 0x7f);
    double a = fabs((double)x);
    if (a < ldexp(1.0, -6)) {                  /* subnormal: units of 2^-9 */
        double q = nearbyint(a * 512.0);       /* q in 0..8, 8 == min normal */
        return (uint8_t)(sign | (uint8_t)q);
    }
    if (isinf(x)) return (uint8_t)(sign | 0x7e);
    int e;
    double m = frexp(a, &e);
    e -= 1; m *= 2.0;
    double q = nearbyint((m - 1.0) * 8.0);
    if (q >= 8.0) { q = 0.0; e += 1; }
    int ef = e + 7;
    if (ef > 15 || (ef == 15 && q >= 7.0)) return (uint8_t)(sign | 0x7e);
    return (uint8_t)(sign | (uint8_t)(ef << 3) | (uint8_t)q);
}

/* OCP 8-bit floating point spec, E5M2: bias 15, IEEE-style inf (S.11111.00)
 * and NaN (S.11111.xx, xx != 0), max finite 57344, subnormals m/4 * 2^-14. */
float bo_e5m2_to_f32(uint8_t b) {
    int s = b >> 7, e = (b >> 2) & 0x1f, m = b & 3;
    double v;
    if (e == 31) v = m ? NAN : INFINITY;
    else if (e == 0) v = ldexp((double)m, -16);
    else v = ldexp(1.0 + m / 4.0, e - 15);
    return (float)(s ? -v : v);
}

/* Saturating RNE encode to E5M2 (baracuda_dtype.cuh:48-57: SATFINITE, so
 * inf and |x| beyond 57344 clamp to max-finite; NaN -> NaN). */
uint8_t bo_f32_to_e5m2_satfinite(float x) {
    uint8_t sign = (f32_bits(x) >> 24) & 0x80u;
    if (isnan(x)) return (uint8_t)(sign | 0x7f);
    double a = fabs((double)x);
    if (a < ldexp(1.0, -14)) {                 /* subnormal: units of 2^-16 */
        double q = nearbyint(a * 65536.0);     /* q in 0..4, 4 == min normal */
        return (uint8_t)(sign | (uint8_t)q);
    }
    if (isinf(x)) return (uint8_t)(sign | 0x7b);
    int e;
    double m = frexp(a, &e);
    e -= 1; m *= 2.0;
    double q = nearbyint((m - 1.0) * 4.0);
    if (q >= 4.0) { q = 0.0; e += 1; }
    int ef = e + 15;
    if (ef > 30) return (uint8_t)(sign | 0x7b);
    return (uint8_t)(sign | (uint8_t)(ef << 2) | (uint8_t)q);
}

/* oracle.rs:922-935 encode_float(.., I32): Rust `f as i32` truncates toward
 * zero, saturates at the i32 range and maps NaN to 0. */
int32_t bo_f64_to_i32_as(double f) {
    if (isnan(f)) return 0;
    if (f >= 2147483647.0) return INT32_MAX;
    if (f <= -2147483648.0) return INT32_MIN;
    return (int32_t)f;
}

/* baracuda_dtype.cuh:23-28 sat_cast_f32_to_s8: round-half-to-even then clamp
 * to [-128,127].  (The smoke test's host twin, int8_smoke.rs:63-66, rounds
 * half away from zero and allows +-1; RNE is the kernel's rule.) */
int8_t bo_sat_cast_s8(float x) {
    if (isnan(x)) return 0;
    double r = nearbyint((double)x);
    if (r < -128.0) r = -128.0;
    if (r > 127.0) r = 127.0;
    return (int8_t)r;
}

/* oracle.rs:1289-1372 eval_contraction, rank-2 case: K ascending, f64
 * accumulator, operands read through physical strides (read_strided,
 * oracle.rs:980-1003), stored through encode_float to I32. */
void bo_contraction_s8_i32(int64_t m, int64_t n, int64_t k,
                           const int8_t *a, int64_t sa0, int64_t sa1,
                           const int8_t *b, int64_t sb0, int64_t sb1,
                           int32_t *out, int64_t ldo) {
    for (int64_t mi = 0; mi < m; ++mi)
        for (int64_t ni = 0; ni < n; ++ni) {
            double acc = 0.0;
            for (int64_t kk = 0; kk < k; ++kk)
                acc += (double)a[mi * sa0 + kk * sa1] * (double)b[kk * sb0 + ni * sb1];
            out[mi * ldo + ni] = bo_f64_to_i32_as(acc);
        }
}

void bo_contraction_f64(int64_t m, int64_t n, int64_t k,
                        const double *a, int64_t sa0, int64_t sa1,
                        const double *b, int64_t sb0, int64_t sb1,
                        double *out, int64_t ldo) {
    for (int64_t mi = 0; mi < m; ++mi)
        for (int64_t ni = 0; ni < n; ++ni) {
            double acc = 0.0;
            for (int64_t kk = 0; kk < k; ++kk)
                acc += a[mi * sa0 + kk * sa1] * b[kk * sb0 + ni * sb1];
            out[mi * ldo + ni] = acc;
        }
}

static int pick_threads(int nthreads) { return nthreads < 1 ? 1 : nthreads; }

/* int8_smoke.rs:85-124 cpu_int_gemm_rcr accumulator (B column-major, read
 * at b[kk + j*ldb]).  Exact integer sum; identical to the saturating i32
 * sum whenever |acc| < 2^31 (always true for |v|<=127, K < 133143). */
void bo_gemm_s8_rcr_i32(int64_t m, int64_t n, int64_t k,
                        const int8_t *a, int64_t lda,
                        const int8_t *b, int64_t ldb,
                        int32_t *d, int64_t ldd,
                        int64_t row0, int64_t row1, int nthreads) {
    (void)m;
    int nt = pick_threads(nthreads);
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
    for (int64_t i = row0; i < row1; ++i) {
        const int8_t *ar = a + i * lda;
        for (int64_t j = 0; j < n; ++j) {
            const int8_t *bc = b + j * ldb;
            int32_t acc = 0;
            for (int64_t kk = 0; kk < k; ++kk) acc += (int32_t)ar[kk] * (int32_t)bc[kk];
            d[i * ldd + j] = acc;
        }
    }
}

/* int8_smoke.rs:85-124 epilogue chain z = alpha*acc + beta*C, then the
 * kernel's sat-cast (RNE + clamp). */
void bo_gemm_s8_rcr_s8(int64_t m, int64_t n, int64_t k,
                       const int8_t *a, int64_t lda,
                       const int8_t *b, int64_t ldb,
                       const int8_t *c, int64_t ldc,
                       int8_t *d, int64_t ldd,
                       float alpha, float beta) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t acc = 0;
            for (int64_t kk = 0; kk < k; ++kk)
                acc += (int64_t)a[i * lda + kk] * (int64_t)b[j * ldb + kk];
            float z = alpha * (float)(int32_t)acc;
            if (c != NULL && beta != 0.0f) z += beta * (float)c[i * ldc + j];
            d[i * ldd + j] = bo_sat_cast_s8(z);
        }
}

/* baracuda_te_shim.cu fused_cast_amax_kernel: out = sat_fp8(v * s) in f32,
 * amax = max |v| with NaN never winning (`av > tmax`). */
void bo_te_cast_amax(const float *x, int64_t n, float scale, int fmt, uint8_t *out, float *amax) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float av = fabsf(x[i]);
        if (av > m) m = av;
        volatile float vs = x[i] * scale;
        out[i] = fmt ? bo_f32_to_e5m2_satfinite(vs) : bo_f32_to_e4m3_satfinite(vs);
    }
    *amax = m;
}

/* baracuda_te_shim.cu dequant_kernel: y = dec(x) * si in f32 (callers round
 * to f16 / bf16 with the RNE codecs above). */
void bo_te_dequant(const uint8_t *x, int64_t n, float scale_inv, int fmt, float *y) {
    for (int64_t i = 0; i < n; ++i) {
        volatile float v = (fmt ? bo_e5m2_to_f32(x[i]) : bo_e4m3_to_f32(x[i])) * scale_inv;
        y[i] = v;
    }
}

/* baracuda_embedding.cuh:61-88 (embedding_kernel), one row at a time. */
void bo_embedding(void *out, const void *weight, const void *idx, int64_t idx_size, int64_t n,
                  int64_t V, int64_t D, int64_t elem_size, int64_t padding_idx) {
    const int64_t rb = D * elem_size;
    for (int64_t r = 0; r < n; ++r) {
        const int64_t v = idx_size == 8 ? ((const int64_t *)idx)[r] : (int64_t)((const int32_t *)idx)[r];
        uint8_t *dst = (uint8_t *)out + r * rb;
        if (v == padding_idx || v < 0 || v >= V) memset(dst, 0, (size_t)rb);
        else memcpy(dst, (const uint8_t *)weight + v * rb, (size_t)rb);
    }
}

/* int8_rrr_smoke.rs:35-48 (erf_approx), f32 arithmetic in the test's order. */
float bo_erf_as7126(float x) {
    const float sign = x < 0.0f ? -1.0f : 1.0f;
    const float ax = fabsf(x);
    const float p = 0.3275911f, a1 = 0.254829592f, a2 = -0.284496736f, a3 = 1.421413741f,
                a4 = -1.453152027f, a5 = 1.061405429f;
    const float t = 1.0f / (1.0f + p * ax);
    const float y = 1.0f - (((((a5 * t + a4) * t) + a3) * t + a2) * t + a1) * t * expf(-ax * ax);
    return sign * y;
}

static float act_apply(int act, float x) {
    switch (act) {
    case 1: return x > 0.0f ? x : 0.0f;                                          /* relu :31-33 */
    case 2: return 0.5f * x * (1.0f + bo_erf_as7126(x * (1.0f / 1.41421356237309504880f))); /* :50-53 */
    case 3: return x / (1.0f + expf(-x));                                        /* silu :55-57 */
    default: return x;
    }
}

/* int8_rrr_smoke.rs:97-131 (cpu_int_gemm_rrr; the RCR twin indexes b[j*ldb+k]).
 * The sum is exact in int64; for |a|,|b| <= 128 and k < 2^17 it equals the
 * reference's saturating i32 sum. */
void bo_gemm_s8_epi(int64_t m, int64_t n, int64_t k,
                    const int8_t *a, int64_t lda,
                    const int8_t *b, int64_t sbk, int64_t sbn,
                    const int8_t *c, int64_t ldc, const float *bias, int act,
                    int8_t *d, int64_t ldd, float alpha, float beta) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t acc = 0;
            for (int64_t kk = 0; kk < k; ++kk)
                acc += (int64_t)a[i * lda + kk] * (int64_t)b[kk * sbk + j * sbn];
            float z = alpha * (float)(int32_t)acc;
            if (c != NULL) z += beta * (float)c[i * ldc + j];
            if (bias != NULL) z += bias[j];
            d[i * ldd + j] = bo_sat_cast_s8(act_apply(act, z));
        }
}

static uint8_t sat_cast_u8(float x) {
    float r = nearbyintf(x);
    if (r < 0.0f) r = 0.0f;
    if (r > 255.0f) r = 255.0f;
    return (uint8_t)(int)r;
}

void bo_gemm_u8_epi(int64_t m, int64_t n, int64_t k,
                    const uint8_t *a, int64_t lda,
                    const uint8_t *b, int64_t sbk, int64_t sbn,
                    const uint8_t *c, int64_t ldc, const float *bias, int act,
                    uint8_t *d, int64_t ldd, float alpha, float beta) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t acc = 0;
            for (int64_t kk = 0; kk < k; ++kk)
                acc += (int64_t)a[i * lda + kk] * (int64_t)b[kk * sbk + j * sbn];
            float z = alpha * (float)(int32_t)acc;
            if (c != NULL) z += beta * (float)c[i * ldc + j];
            if (bias != NULL) z += bias[j];
            d[i * ldd + j] = sat_cast_u8(act_apply(act, z));
        }
}

/* baracuda_quantize_compose.cuh:265-274: y = sa*sw*(float)acc, evaluated
 * left to right in f32, i.e. (sa*sw)*acc; the bf16 store is oracle.rs:397-404. */
void bo_gemm_w8a8_rcr_bf16(int64_t m, int64_t n, int64_t k,
                           const int8_t *a, int64_t lda,
                           const int8_t *w, int64_t ldw,
                           const float *sa, const float *sw,
                           uint16_t *d, int64_t ldd,
                           int64_t row0, int64_t row1, int nthreads) {
    (void)m;
    int nt = pick_threads(nthreads);
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
    for (int64_t i = row0; i < row1; ++i) {
        const int8_t *ar = a + i * lda;
        for (int64_t j = 0; j < n; ++j) {
            const int8_t *wr = w + j * ldw;
            int32_t acc = 0;
            for (int64_t kk = 0; kk < k; ++kk) acc += (int32_t)ar[kk] * (int32_t)wr[kk];
            volatile float s = sa[i] * sw[j];   /* keep the f32 rounding of the product */
            float y = s * (float)acc;
            d[i * ldd + j] = bo_f32_to_bf16_bits(y);
        }
    }
}

void bo_gemm_fp8_e4m3_rcr_f64(int64_t m, int64_t n, int64_t k,
                              const uint8_t *a, int64_t lda,
                              const uint8_t *b, int64_t ldb,
                              double *acc, int64_t ldacc,
                              int64_t row0, int64_t row1, int nthreads) {
    (void)m;
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = bo_e4m3_to_f32((uint8_t)i);
    int nt = pick_threads(nthreads);
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
    for (int64_t i = row0; i < row1; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double s = 0.0;
            for (int64_t kk = 0; kk < k; ++kk)
                s += (double)lut[a[i * lda + kk]] * (double)lut[b[j * ldb + kk]];
            acc[i * ldacc + j] = s;
        }
}

/* FP8 GEMM exact accumulator, either encoding (fmt 0 e4m3, 1 e5m2) and
 * either B layout (b[k,j] at b[k*sbk + j*sbn]); the products and the sum are
 * exact in f64 for every K used here. */
void bo_gemm_fp8_f64(int fmt, int64_t m, int64_t n, int64_t k,
                     const uint8_t *a, int64_t lda, const uint8_t *b, int64_t sbk, int64_t sbn,
                     double *acc, int64_t ldacc, int64_t row0, int64_t row1, int nthreads) {
    (void)m;
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = fmt ? bo_e5m2_to_f32((uint8_t)i) : bo_e4m3_to_f32((uint8_t)i);
    int nt = pick_threads(nthreads);
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
    for (int64_t i = row0; i < row1; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double s = 0.0;
            for (int64_t kk = 0; kk < k; ++kk)
                s += (double)lut[a[i * lda + kk]] * (double)lut[b[kk * sbk + j * sbn]];
            acc[(i - row0) * ldacc + j] = s;
        }
}

/* FP8-out epilogue of gemm_fp8_{rcr,rrr}_sm89 (baracuda_fp8_rrr_sm89.cuh:190-235,
 * fp8_bias_smoke.rs:125-160):
 *   z = alpha*(f32)acc [+ beta*dec(C)] [+ bias[j]] ; D = sat_fp8(act(z))
 * acc is the exact sum rounded once to f32. */
void bo_fp8_epilogue(int fmt, int64_t m, int64_t n, const double *acc, int64_t ldacc,
                     const uint8_t *c, int64_t ldc, const float *bias, int act,
                     float alpha, float beta, uint8_t *d, int64_t ldd) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float z = alpha * (float)acc[i * ldacc + j];
            if (c != NULL) z += beta * (fmt ? bo_e5m2_to_f32(c[i * ldc + j]) : bo_e4m3_to_f32(c[i * ldc + j]));
            if (bias != NULL) z += bias[j];
            z = act_apply(act, z);
            d[i * ldd + j] = fmt ? bo_f32_to_e5m2_satfinite(z) : bo_f32_to_e4m3_satfinite(z);
        }
}

/* fp8_e4m3_rcr_smoke.rs:51-76 cpu_fp8_e4m3_gemm_rcr: f32 accumulator, K
 * ascending, B column-major at b[j*ldb + kk]. */
void bo_gemm_fp8_e4m3_rcr_f32(int64_t m, int64_t n, int64_t k,
                              const uint8_t *a, int64_t lda,
                              const uint8_t *b, int64_t ldb,
                              float *acc, int64_t ldacc) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float s = 0.0f;
            for (int64_t kk = 0; kk < k; ++kk) {
                volatile float p = bo_e4m3_to_f32(a[i * lda + kk]) * bo_e4m3_to_f32(b[j * ldb + kk]);
                s += p;
            }
            acc[i * ldacc + j] = s;
        }
}

/* gemv_dense_smoke.rs:45-75 cpu_gemv (f64, RRR, strided batch). */
void bo_gemv_dense_m1_f64(int64_t n, int64_t k, int64_t batch,
                          const double *a, int64_t stride_a,
                          const double *b, int64_t ldb, int64_t stride_b,
                          const double *d_init, double *d, int64_t stride_d,
                          double alpha, double beta) {
    for (int64_t g = 0; g < batch; ++g) {
        const double *a0 = a + g * stride_a;
        const double *b0 = b + g * stride_b;
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (int64_t kk = 0; kk < k; ++kk) acc += a0[kk] * b0[kk * ldb + j];
            d[g * stride_d + j] = alpha * acc + beta * d_init[g * stride_d + j];
        }
    }
}

/* int8 weight-only decode GEMV (new SKU; semantics of gemv_dense.cu:148-170
 * with B = W^T stored [N,K] and a per-row scale): f64 dot product. */
void bo_gemv_s8w_m1_f64(int64_t n, int64_t k,
                        const uint16_t *x_bf16, const int8_t *w, int64_t ldw,
                        double *acc, int nthreads) {
    float *x = (float *)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
    for (int64_t kk = 0; kk < k; ++kk) x[kk] = bo_bf16_bits_to_f32(x_bf16[kk]);
    int nt = pick_threads(nthreads);
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
    for (int64_t j = 0; j < n; ++j) {
        const int8_t *wr = w + j * ldw;
        double s = 0.0;
        for (int64_t kk = 0; kk < k; ++kk) s += (double)x[kk] * (double)wr[kk];
        acc[j] = s;
    }
    free(x);
}

/* gather_rows.cu:60-84: every output element written; idx >= V -> zero. */
void bo_gather_rows(void *dest, const void *table, const uint32_t *idx,
                    int64_t V, int64_t H, int64_t n, int64_t elem_size) {
    size_t row_bytes = (size_t)(H * elem_size);
    for (int64_t r = 0; r < n; ++r) {
        uint8_t *dst = (uint8_t *)dest + (size_t)r * row_bytes;
        if ((int64_t)idx[r] < V)
            memcpy(dst, (const uint8_t *)table + (size_t)idx[r] * row_bytes, row_bytes);
        else
            memset(dst, 0, row_bytes);
    }
}

/* baracuda_quantize_compose.cuh:143-203 dynamic_range_quantize_per_token_
 * symmetric_kernel: max-abs over the row (NaN ignored by the `a > max`
 * compare), scale = max/qmax (1 if max == 0), inv = 1/scale, then
 * q = clamp(rne(x*inv)) cast to int8 (__float2int_rn(NaN) = 0). All in f32. */
void bo_quantize_per_token_sym(const float *x, int64_t n, int64_t d, int32_t qmin,
                               int32_t qmax, float *scale, int8_t *q) {
    for (int64_t r = 0; r < n; ++r) {
        const float *row = x + r * d;
        float m = 0.0f;
        for (int64_t c = 0; c < d; ++c) {
            float a = fabsf(row[c]);
            if (a > m) m = a;
        }
        volatile float s = m > 0.0f ? m / (float)qmax : 1.0f;
        volatile float inv = s != 0.0f ? 1.0f / s : 0.0f;
        scale[r] = s;
        for (int64_t c = 0; c < d; ++c) {
            volatile float p = row[c] * inv;
            int32_t v = isnan(p) ? 0 : (int32_t)nearbyintf(p);
            if (isnan(p)) v = 0;
            if (v < qmin) v = qmin;
            if (v > qmax) v = qmax;
            q[r * d + c] = (int8_t)v;
        }
    }
}

/* baracuda_moe.cuh:1121-1162: histogram of expert_ids, then exclusive
 * prefix sum into offsets[0..E], offsets[0] = 0.  Ids outside [0, E) are
 * not counted: the reference indexes its counters with them (out of
 * bounds); the GPU offsets kernel skips them, and so does this restatement. */
void bo_moe_expert_offsets(const int32_t *expert_ids, int64_t size_m,
                           int32_t num_experts, int32_t *counts,
                           int32_t *offsets) {
    for (int32_t e = 0; e < num_experts; ++e) counts[e] = 0;
    for (int64_t i = 0; i < size_m; ++i)
        if (expert_ids[i] >= 0 && expert_ids[i] < num_experts) counts[expert_ids[i]] += 1;
    offsets[0] = 0;
    for (int32_t e = 0; e < num_experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
}

/* baracuda_moe.cuh:827-944 moe_gemm_wmma_kernel routing, int8 operands,
 * topk_weights == NULL form: input row = pair / topk, output row = pair. */
void bo_moe_s8_grouped_i32(const int8_t *x, const int8_t *w,
                           const int32_t *sorted_token_ids,
                           const int32_t *offsets, int32_t num_experts,
                           int32_t topk, int64_t size_m, int64_t n,
                           int64_t k, int32_t *acc_out) {
    for (int32_t e = 0; e < num_experts; ++e) {
        const int8_t *we = w + (int64_t)e * n * k;
        for (int32_t p = offsets[e]; p < offsets[e + 1]; ++p) {
            if (p >= size_m) continue;
            int32_t tok = sorted_token_ids[p];
            const int8_t *xr = x + (int64_t)(tok / topk) * k;
            for (int64_t j = 0; j < n; ++j) {
                const int8_t *wr = we + j * k;
                int32_t acc = 0;
                for (int64_t kk = 0; kk < k; ++kk) acc += (int32_t)xr[kk] * (int32_t)wr[kk];
                acc_out[(int64_t)tok * n + j] = acc;
            }
        }
    }
}

/* baracuda_moe.cuh:827-944: the float (WMMA) MoE GEMM restated in f64. */
void bo_moe_grouped_f64(const float *x, const float *w, const int32_t *sorted_token_ids,
                        const int32_t *offsets, int32_t num_experts, int32_t topk,
                        const float *topk_w, int64_t n, int64_t k, double *out) {
    for (int32_t e = 0; e < num_experts; ++e)
        for (int32_t p = offsets[e]; p < offsets[e + 1]; ++p) {
            const int64_t tok = sorted_token_ids[p];
            const int64_t in_row = topk_w ? tok : tok / topk;
            const double tw = topk_w ? (double)topk_w[tok] : 1.0;
            for (int64_t j = 0; j < n; ++j) {
                double acc = 0.0;
                for (int64_t kk = 0; kk < k; ++kk)
                    acc += (double)x[in_row * k + kk] * (double)w[((int64_t)e * n + j) * k + kk];
                out[tok * n + j] = acc * tw;
            }
        }
}
