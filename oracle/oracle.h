/*
 * oracle.h -- CPU restatement of baracuda's reference arithmetic for the
 * quantized-inference contraction path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product (baracuda_amd/, libbaracuda_kernels.so) never links or
 * calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the baracuda repository root).  How each function is
 * pinned (golden vectors, closed forms, library cross-checks) is recorded in
 * tests/test_oracle.py next to the pin itself.
 */
#ifndef BARACUDA_ORACLE_H
#define BARACUDA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs ----------------------------------------------------- */
uint16_t bo_f32_to_bf16_bits(float x);
float    bo_bf16_bits_to_f32(uint16_t b);
uint16_t bo_f32_to_f16_bits(float x);
float    bo_f16_bits_to_f32(uint16_t h);
float    bo_e4m3_to_f32(uint8_t b);
uint8_t  bo_f32_to_e4m3_satfinite(float x);
float    bo_e5m2_to_f32(uint8_t b);
uint8_t  bo_f32_to_e5m2_satfinite(float x);
int32_t  bo_f64_to_i32_as(double f);     /* Rust `f as i32` (saturating, NaN->0) */
int8_t   bo_sat_cast_s8(float x);        /* RNE + clamp to [-128,127]            */

/* ---- contractions ------------------------------------------------------ */
/* oracle.rs eval_contraction restated for int8 operands read as I32:
 * out[m*ldo+n] = (i32)( sum_{k ascending} (f64)a[m*sa0+k*sa1] * (f64)b[k*sb0+n*sb1] ) */
void bo_contraction_s8_i32(int64_t m, int64_t n, int64_t k,
                           const int8_t *a, int64_t sa0, int64_t sa1,
                           const int8_t *b, int64_t sb0, int64_t sb1,
                           int32_t *out, int64_t ldo);
/* Same over f64 operands (the oracle's own hand-computed test uses f32/f64). */
void bo_contraction_f64(int64_t m, int64_t n, int64_t k,
                        const double *a, int64_t sa0, int64_t sa1,
                        const double *b, int64_t sb0, int64_t sb1,
                        double *out, int64_t ldo);

/* int32 RCR accumulator, exact integer arithmetic (int64 sum).  Rows
 * [row0,row1) only, so a bounded sample can be timed. nthreads<=1 = serial. */
void bo_gemm_s8_rcr_i32(int64_t m, int64_t n, int64_t k,
                        const int8_t *a, int64_t lda,
                        const int8_t *b, int64_t ldb,
                        int32_t *d, int64_t ldd,
                        int64_t row0, int64_t row1, int nthreads);

/* int8 GEMM with the int8-out epilogue of cpu_int_gemm_rcr:
 * z = alpha*(f32)acc + beta*(f32)C ; D = sat_cast_s8(z).  c may be NULL. */
void bo_gemm_s8_rcr_s8(int64_t m, int64_t n, int64_t k,
                       const int8_t *a, int64_t lda,
                       const int8_t *b, int64_t ldb,
                       const int8_t *c, int64_t ldc,
                       int8_t *d, int64_t ldd,
                       float alpha, float beta);

/* int8-out GEMM with the bias / activation epilogue of the reference's RRR
 * and RCR smoke tests (crates/baracuda-kernels/tests/int8_rrr_smoke.rs:31-131):
 *   acc = sum_k a[i,k]*b[k,j]   with b[k,j] at b[k*sbk + j*sbn]
 *   z   = alpha*(f32)acc + beta*(f32)C[i,j] (when c) + bias[j] (when bias)
 *   D   = sat_cast_s8(act(z))
 * act: 0 none, 1 relu, 2 gelu (erf via Abramowitz-Stegun 7.1.26), 3 silu.
 * Bias is passed as f32 (an i32 bias converts exactly for |bias| < 2^24). */
void bo_gemm_s8_epi(int64_t m, int64_t n, int64_t k,
                    const int8_t *a, int64_t lda,
                    const int8_t *b, int64_t sbk, int64_t sbn,
                    const int8_t *c, int64_t ldc, const float *bias, int act,
                    int8_t *d, int64_t ldd, float alpha, float beta);
float bo_erf_as7126(float x);
/* The same for u8 operands / C / D (gemm_u8_rrr_sm80: sat_cast_u8 = RNE +
 * clamp to [0, 255], int8_rrr_smoke.rs:79-81). */
void bo_gemm_u8_epi(int64_t m, int64_t n, int64_t k,
                    const uint8_t *a, int64_t lda,
                    const uint8_t *b, int64_t sbk, int64_t sbn,
                    const uint8_t *c, int64_t ldc, const float *bias, int act,
                    uint8_t *d, int64_t ldd, float alpha, float beta);

/* W8A8: out = bf16( (sa[m]*sw[n]) * (f32)acc ) with f32 products. */
void bo_gemm_w8a8_rcr_bf16(int64_t m, int64_t n, int64_t k,
                           const int8_t *a, int64_t lda,
                           const int8_t *w, int64_t ldw,
                           const float *sa, const float *sw,
                           uint16_t *d, int64_t ldd,
                           int64_t row0, int64_t row1, int nthreads);

/* FP8 e4m3 RCR: acc = sum_k dec(a)*dec(b) in f64 (exact reference value),
 * written as f64; callers derive bf16 / e4m3 / f32 outputs from it. */
void bo_gemm_fp8_e4m3_rcr_f64(int64_t m, int64_t n, int64_t k,
                              const uint8_t *a, int64_t lda,
                              const uint8_t *b, int64_t ldb,
                              double *acc, int64_t ldacc,
                              int64_t row0, int64_t row1, int nthreads);
/* Either encoding (fmt 0 e4m3, 1 e5m2) and layout (b[k,j] at b[k*sbk+j*sbn]);
 * rows [row0,row1) written from acc row 0. */
void bo_gemm_fp8_f64(int fmt, int64_t m, int64_t n, int64_t k,
                     const uint8_t *a, int64_t lda, const uint8_t *b, int64_t sbk, int64_t sbn,
                     double *acc, int64_t ldacc, int64_t row0, int64_t row1, int nthreads);
/* FP8-out epilogue: D = sat_fp8(act(alpha*(f32)acc + beta*dec(C) + bias)),
 * c / bias may be NULL; act as in bo_gemm_s8_epi. */
void bo_fp8_epilogue(int fmt, int64_t m, int64_t n, const double *acc, int64_t ldacc,
                     const uint8_t *c, int64_t ldc, const float *bias, int act,
                     float alpha, float beta, uint8_t *d, int64_t ldd);
/* The reference smoke test's own f32 K-ascending accumulation. */
void bo_gemm_fp8_e4m3_rcr_f32(int64_t m, int64_t n, int64_t k,
                              const uint8_t *a, int64_t lda,
                              const uint8_t *b, int64_t ldb,
                              float *acc, int64_t ldacc);

/* gemv_dense_m1 f64 reference (RRR):
 * D[g,j] = alpha*sum_k A[g,k]*B[g,k,j] + beta*Dinit[g,j] */
void bo_gemv_dense_m1_f64(int64_t n, int64_t k, int64_t batch,
                          const double *a, int64_t stride_a,
                          const double *b, int64_t ldb, int64_t stride_b,
                          const double *d_init, double *d, int64_t stride_d,
                          double alpha, double beta);

/* int8 weight-only m=1 GEMV: acc[n] = sum_k x[k]*w[n,k] (f64), out in f64
 * before scale; caller applies scale/bf16. x given as bf16 bits. */
void bo_gemv_s8w_m1_f64(int64_t n, int64_t k,
                        const uint16_t *x_bf16, const int8_t *w, int64_t ldw,
                        double *acc, int nthreads);

/* gather_rows: dest[r,:] = table[idx[r],:], zero when idx[r] >= V.
 * elem_size in bytes (2 or 4). */
void bo_gather_rows(void *dest, const void *table, const uint32_t *idx,
                    int64_t V, int64_t H, int64_t n, int64_t elem_size);

/* FP8 delayed-scaling quantizer (baracuda_te_shim.cu fused_cast_amax_kernel,
 * dequant_kernel): x widened to f32 by the caller. */
void bo_te_cast_amax(const float *x, int64_t n, float scale, int fmt, uint8_t *out, float *amax);
void bo_te_dequant(const uint8_t *x, int64_t n, float scale_inv, int fmt, float *y);

/* embedding forward (baracuda_embedding.cuh:61-88): out[r,:] = weight[idx[r],:],
 * zero when idx[r] == padding_idx, idx[r] < 0 or idx[r] >= V.  idx_size 4
 * (i32) or 8 (i64); elem_size in bytes. */
void bo_embedding(void *out, const void *weight, const void *idx, int64_t idx_size, int64_t n,
                  int64_t V, int64_t D, int64_t elem_size, int64_t padding_idx);

/* dynamic_range_quantize_per_token_sym (baracuda_quantize_compose.cuh:143-203):
 * x given as f32 (callers narrow f64 / widen bf16 first, like qc_load_as_f32). */
void bo_quantize_per_token_sym(const float *x, int64_t n, int64_t d, int32_t qmin,
                               int32_t qmax, float *scale, int8_t *q);

/* MoE routing helpers (baracuda_moe.cuh:1121-1162). */
void bo_moe_expert_offsets(const int32_t *expert_ids, int64_t size_m,
                           int32_t num_experts, int32_t *counts,
                           int32_t *offsets);
/* Grouped int8 expert GEMM, int32 accumulators, row = sorted pair:
 *   for each segment e, pair p in it: tok = sorted_token_ids[p],
 *   in_row = tok / topk ; acc[tok, n] = sum_k x[in_row,k]*w[e,n,k]. */
void bo_moe_s8_grouped_i32(const int8_t *x, const int8_t *w,
                           const int32_t *sorted_token_ids,
                           const int32_t *offsets, int32_t num_experts,
                           int32_t topk, int64_t size_m, int64_t n,
                           int64_t k, int32_t *acc_out);

/* Float MoE (baracuda_moe.cuh:827-944, moe_gemm_wmma_kernel): for each
 * segment e and pair p in it: tok = sorted_token_ids[p],
 * in_row = topk_w ? tok : tok / topk,
 * out[tok, n] = (topk_w ? topk_w[tok] : 1) * sum_k x[in_row,k]*w[e,n,k] in f64
 * (inputs given as f32, decoded from bf16/f16 by the caller). */
void bo_moe_grouped_f64(const float *x, const float *w, const int32_t *sorted_token_ids,
                        const int32_t *offsets, int32_t num_experts, int32_t topk,
                        const float *topk_w, int64_t n, int64_t k, double *out);

#ifdef __cplusplus
}
#endif
#endif
