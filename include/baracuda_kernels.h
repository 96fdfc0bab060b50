/*
 * baracuda_kernels.h -- C ABI of the MI355X (gfx950) quantized-inference
 * contraction path: a drop-in for the corresponding baracuda-kernels-sys
 * entry points.
 *
 * Conventions (crates/baracuda-kernels-sys/src/lib.rs:10-27, ARCHITECTURE.md:253-375
 * of the reference):
 *   - status: 0 ok, 1 misaligned, 2 invalid problem, 3 unsupported,
 *             4 workspace too small, 5 launch failure;
 *   - all pointers are device pointers owned by the caller; nothing here
 *     allocates, frees, memsets or synchronises, so every _run can be
 *     captured into a hipGraph;
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream);
 *   - strides and leading dimensions are in elements;
 *   - workspace is never required: every _workspace_size returns 0 except
 *     the u8 RRR family's, gemv_dense_m1's (large shapes) and the int8 RCR
 *     SKUs' (s8 / i32 / W8A8 bf16 out and the bias family, when the last
 *     round of 256 x 256 tiles on the 256 CUs is at most half full and the
 *     last rows are not a streamed pass: M % 256 in [1, 64] whose row of
 *     tiles would start another round, or M <= 64, runs its last rows as a
 *     second launch without any workspace; 65..128 such rows do so when no
 *     workspace is passed), whose
 *     optional workspace (when given at least that size, 256- / 16-byte
 *     aligned; contents on entry do not matter) selects a faster path: the
 *     u8 pre-pass, the dense GEMV's split-K, the int8 tail round split along
 *     K (two launches, bit-identical output).  Without it every entry point
 *     runs as-is.
 *
 * Each declaration cites the reference entry point it replaces
 * (paths relative to the baracuda repository root).
 */
#ifndef BARACUDA_KERNELS_GFX950_H
#define BARACUDA_KERNELS_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================= int8 GEMM, RCR layout ===========================
 * A row-major [M,K] (lda), B column-major [K,N] = row-major [N,K] (ldb),
 * int32 accumulator (wraps mod 2^32; equals the reference's saturating
 * accumulator whenever |acc| < 2^31, e.g. |a|,|b| <= 127 and K < 133143). */

/* Replaces baracuda_kernels_gemm_s8_rcr_sm80_{run,workspace_size,can_implement}
 * (crates/baracuda-kernels-sys/src/cutlass_reexport.rs:661-666,
 *  crates/baracuda-cutlass-kernels-sys/kernels/gemm_s8_rcr_sm80.cu:169-198):
 * D = sat_s8(rne(alpha*acc + beta*C)).  A NULL C means C = D with ldc = ldd
 * (the CUTLASS kernel's c_eff, gemm_s8_rcr_sm80.cu:87-89): beta != 0 then
 * accumulates into D in place.  The same holds for the RCR bias family and
 * the u8 RCR SKUs below; the RRR SKUs skip the beta term for a NULL C. */
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_s8_rcr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd);

/* New SKU (same family): D = acc as int32 [M,N] (ldd).  The plain int8
 * contraction of kernelgen's oracle (crates/baracuda-kernelgen/src/oracle.rs:1289-1372)
 * evaluated on the device. */
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    void *d, int64_t ldd, void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd);

/* New SKU: W8A8 per-token x per-channel dequant to bf16,
 * D[m,n] = bf16_rne((scale_a[m] * scale_b[n]) * (float)acc), the
 * quantized_linear_w8a8 epilogue order
 * (crates/baracuda-kernels-sys/kernels/include/baracuda_quantize_compose.cuh:265-274). */
int32_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const float *scale_a, const float *scale_b, void *d, int64_t ldd,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *scale_a, const void *scale_b, const void *d, int64_t ldd);

/* Replaces baracuda_kernels_quantized_linear_w8a8_f32_{run,can_implement}
 * (baracuda_quantize_compose.cuh:340-370, crates/baracuda-kernels-sys/src/lib.rs:64915,64963):
 * output[M,C_out] f32 = scale_a[m]*scale_w[c]*acc, weight [C_out,K], act [M,K]. */
int32_t baracuda_kernels_quantized_linear_w8a8_f32_gfx950_run(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, void *output,
    void *workspace, size_t workspace_bytes, void *stream);
int32_t baracuda_kernels_quantized_linear_w8a8_f32_gfx950_can_implement(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, const void *output);

/* Replaces baracuda_kernels_quantized_linear_w8a8_f64_{run,can_implement}
 * (crates/baracuda-kernels-sys/kernels/quantize/compose.cu:27-28, macro at
 * baracuda_quantize_compose.cuh:340-370): f64 scale_a [M], scale_w [C_out] and
 * output [M,C_out]; output = (double)(((float)scale_a[m]*(float)scale_w[c]) * (float)acc),
 * the reference's f32 evaluation with narrowed scales. */
int32_t baracuda_kernels_quantized_linear_w8a8_f64_gfx950_run(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, void *output,
    void *workspace, size_t workspace_bytes, void *stream);
int32_t baracuda_kernels_quantized_linear_w8a8_f64_gfx950_can_implement(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, const void *output);

/* int8 RCR with the bias / activation epilogue family.  Same ABI as
 * baracuda_kernels_gemm_{bias,bias_relu,bias_gelu,bias_silu}_{f32bias,i32bias}_s8_rcr_sm80_*
 * (crates/baracuda-cutlass-kernels-sys/kernels/gemm_s8_rcr_sm80_bias.cu:225-275,
 *  crates/baracuda-kernels-sys/src/cutlass_reexport.rs:1025-):
 * D = sat_s8(rne(act(alpha*acc + beta*C + bias[n]))), act in {identity, relu,
 * gelu (erf), silu}, bias f32 or i32 [N]. */
#define BK_S8_RCR_BIAS_DECL(EPI, BIAS)                                                          \
    int32_t baracuda_kernels_gemm_##EPI##_##BIAS##_s8_rcr_gfx950_run(                           \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha,         \
        float beta, void *workspace, size_t workspace_bytes, void *stream);                      \
    size_t baracuda_kernels_gemm_##EPI##_##BIAS##_s8_rcr_gfx950_workspace_size(int32_t m,       \
                                                                             int32_t n, int32_t k); \
    int32_t baracuda_kernels_gemm_##EPI##_##BIAS##_s8_rcr_gfx950_can_implement(                 \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias);
BK_S8_RCR_BIAS_DECL(bias, f32bias)
BK_S8_RCR_BIAS_DECL(bias_relu, f32bias)
BK_S8_RCR_BIAS_DECL(bias_gelu, f32bias)
BK_S8_RCR_BIAS_DECL(bias_silu, f32bias)
BK_S8_RCR_BIAS_DECL(bias, i32bias)
BK_S8_RCR_BIAS_DECL(bias_relu, i32bias)
BK_S8_RCR_BIAS_DECL(bias_gelu, i32bias)
BK_S8_RCR_BIAS_DECL(bias_silu, i32bias)
#undef BK_S8_RCR_BIAS_DECL

/* ======================= u8 GEMM, RCR layout ============================
 * u8 x u8, A row-major [M,K], B [N,K] (column-major [K,N]), int32 accumulator,
 * D = sat_u8(rne(act(alpha*acc + beta*C [+ bias[n]]))) with C and D u8.
 * Replaces baracuda_kernels_gemm_u8_rcr_sm80_{run,workspace_size,can_implement}
 * (crates/baracuda-cutlass-kernels-sys/kernels/gemm_u8_rcr_sm80.cu; re-exported at
 *  crates/baracuda-kernels-sys/src/cutlass_reexport.rs:669-676) and
 * baracuda_kernels_gemm_{bias,bias_relu,bias_gelu,bias_silu}_{f32bias,i32bias}_u8_rcr_sm80_*
 * (gemm_u8_rcr_sm80_bias.cu; cutlass_reexport.rs:1062-1096, 1141-1176).
 * Workspace 0.  A NULL C reads D in place (gemm_u8_rcr_sm80.cu:77-79). */
int32_t baracuda_kernels_gemm_u8_rcr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_u8_rcr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_u8_rcr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd);
#define BK_U8_RCR_BIAS_DECL(EPI, BIAS)                                                          \
    int32_t baracuda_kernels_gemm_##EPI##_##BIAS##_u8_rcr_gfx950_run(                           \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha,         \
        float beta, void *workspace, size_t workspace_bytes, void *stream);                      \
    size_t baracuda_kernels_gemm_##EPI##_##BIAS##_u8_rcr_gfx950_workspace_size(int32_t m,       \
                                                                             int32_t n, int32_t k); \
    int32_t baracuda_kernels_gemm_##EPI##_##BIAS##_u8_rcr_gfx950_can_implement(                 \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias);
BK_U8_RCR_BIAS_DECL(bias, f32bias)
BK_U8_RCR_BIAS_DECL(bias_relu, f32bias)
BK_U8_RCR_BIAS_DECL(bias_gelu, f32bias)
BK_U8_RCR_BIAS_DECL(bias_silu, f32bias)
BK_U8_RCR_BIAS_DECL(bias, i32bias)
BK_U8_RCR_BIAS_DECL(bias_relu, i32bias)
BK_U8_RCR_BIAS_DECL(bias_gelu, i32bias)
BK_U8_RCR_BIAS_DECL(bias_silu, i32bias)
#undef BK_U8_RCR_BIAS_DECL

/* ======================= int8 GEMM, RRR layout ===========================
 * A row-major [M,K] (lda), B row-major [K,N] (ldb), D row-major [M,N].
 * Replaces baracuda_kernels_gemm_s8_rrr_sm80_{run,workspace_size,can_implement}
 * (crates/baracuda-kernels-sys/kernels/gemm/gemm_s8_rrr_sm80.cu:28-64):
 * D = sat_s8(rne(alpha*acc + beta*C)). */
int32_t baracuda_kernels_gemm_s8_rrr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_s8_rrr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_s8_rrr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd);

/* RRR bias / activation family.  Same ABI as
 * baracuda_kernels_gemm_s8_rrr_sm80_{bias,bias_relu,bias_gelu,bias_silu}_{f32,i32}_{run,can_implement}
 * (crates/baracuda-kernels-sys/kernels/gemm/gemm_s8_rrr_sm80_bias.cu:48-267). */
#define BK_S8_RRR_BIAS_DECL(EPI, BIAS)                                                          \
    int32_t baracuda_kernels_gemm_s8_rrr_gfx950_##EPI##_##BIAS##_run(                           \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha,         \
        float beta, void *workspace, size_t workspace_bytes, void *stream);                      \
    int32_t baracuda_kernels_gemm_s8_rrr_gfx950_##EPI##_##BIAS##_can_implement(                 \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, const void *d, int64_t ldd);
BK_S8_RRR_BIAS_DECL(bias, f32)
BK_S8_RRR_BIAS_DECL(bias_relu, f32)
BK_S8_RRR_BIAS_DECL(bias_gelu, f32)
BK_S8_RRR_BIAS_DECL(bias_silu, f32)
BK_S8_RRR_BIAS_DECL(bias, i32)
BK_S8_RRR_BIAS_DECL(bias_relu, i32)
BK_S8_RRR_BIAS_DECL(bias_gelu, i32)
BK_S8_RRR_BIAS_DECL(bias_silu, i32)
#undef BK_S8_RRR_BIAS_DECL

/* FP8 fp8-out SKUs in both encodings and layouts (B [N,K] for rcr, row-major
 * [K,N] for rrr), D = sat_fp8(alpha*acc + beta*dequant(C)).  Same ABI as
 * baracuda_kernels_gemm_fp8_{e4m3,e5m2}_{rcr,rrr}_sm89_{run,workspace_size,can_implement}
 * (crates/baracuda-kernels-sys/kernels/gemm/gemm_fp8_{e4m3,e5m2}_{rcr,rrr}_sm89.cu). */
#define BK_FP8_DECL(ENC, LAY)                                                                   \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_run(                               \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,               \
        void *workspace, size_t workspace_bytes, void *stream);                                  \
    size_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_workspace_size(int32_t m, int32_t n, \
                                                                          int32_t k);           \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_can_implement(                     \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, const void *d, int64_t ldd);
BK_FP8_DECL(e4m3, rrr)
BK_FP8_DECL(e5m2, rcr)
BK_FP8_DECL(e5m2, rrr)
#undef BK_FP8_DECL

/* FP8 bias / activation family: D = sat_fp8(act(alpha*acc + beta*dequant(C) +
 * bias[n])), bias f32 [N].  Same ABI as
 * baracuda_kernels_gemm_fp8_{e4m3,e5m2}_{rcr,rrr}_sm89_{bias,bias_relu,bias_gelu,bias_silu}_*
 * (crates/baracuda-kernels-sys/kernels/gemm/gemm_fp8_*_sm89_bias.cu,
 *  crates/baracuda-kernels-sys/src/lib.rs:964-1460). */
#define BK_FP8_BIAS_DECL(ENC, LAY, EPI)                                                         \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_##EPI##_run(                       \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha,         \
        float beta, void *workspace, size_t workspace_bytes, void *stream);                      \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_##EPI##_can_implement(             \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, const void *d, int64_t ldd);
#define BK_FP8_BIAS_DECL4(ENC, LAY)                                                             \
    BK_FP8_BIAS_DECL(ENC, LAY, bias)                                                            \
    BK_FP8_BIAS_DECL(ENC, LAY, bias_relu)                                                       \
    BK_FP8_BIAS_DECL(ENC, LAY, bias_gelu)                                                       \
    BK_FP8_BIAS_DECL(ENC, LAY, bias_silu)
BK_FP8_BIAS_DECL4(e4m3, rcr)
BK_FP8_BIAS_DECL4(e4m3, rrr)
BK_FP8_BIAS_DECL4(e5m2, rcr)
BK_FP8_BIAS_DECL4(e5m2, rrr)
#undef BK_FP8_BIAS_DECL4
#undef BK_FP8_BIAS_DECL

/* ======================= u8 GEMM, RRR layout ============================
 * u8 x u8, int32 accumulator, D = sat_u8(rne(act(alpha*acc + beta*C [+ bias])))
 * with C and D u8.  Replaces baracuda_kernels_gemm_u8_rrr_sm80_{run,workspace_size,
 * can_implement} and baracuda_kernels_gemm_u8_rrr_sm80_{bias,...}_{f32,i32}_*
 * (crates/baracuda-kernels-sys/kernels/gemm/gemm_u8_rrr_sm80{,_bias}.cu;
 *  crates/baracuda-kernels-sys/src/lib.rs:120-160, 462-).
 * Optional workspace (all u8 RRR SKUs; its size from
 * baracuda_kernels_gemm_u8_rrr_gfx950_workspace_size, nonzero for whole
 * 256x256 tiles and K % 128 == 0): M*K + K*N bytes of operands flipped to
 * u - 128 plus (M + N) int32 operand sums, written by a pre-pass; contents on
 * entry do not matter.  Without it the flip and the sums run inside the GEMM
 * loop. */
int32_t baracuda_kernels_gemm_u8_rrr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_u8_rrr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_u8_rrr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd);
/* Allocation-free variant of baracuda_kernels_gemm_u8_rrr_gfx950_run (no
 * counterpart in the reference): for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc), which therefore cannot hand in the optional workspace.
 * Whole-tile problems (M, N % 256 == 0, K % 128 == 0, 16-byte aligned
 * operands) use a fixed device array of BARACUDA_U8_RRR_NOALLOC_SCRATCH_BYTES
 * bytes held by each GPU the library runs on until the process ends; a
 * problem whose pre-pass needs more (workspace_size(m, n, k) bytes) returns
 * 4.  Other shapes run the in-loop path.  Calls no hipMalloc,
 * hipFree or allocating routine; every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (different streams, or host
 * threads) race -- serialise them.  Results are identical to
 * baracuda_kernels_gemm_u8_rrr_gfx950_run. */
/* The array is part of the library's code object: every process that loads
 * the library holds this many bytes of device memory on each GPU it uses,
 * whether or not it calls this entry point.  A build may set another size
 * with -DBARACUDA_U8_RRR_NOALLOC_SCRATCH_BYTES=<bytes> (BK_NOALLOC_SCRATCH_MIB
 * for baracuda_amd/build.py).  The array's device address is looked up once
 * per device and kept: hipDeviceReset is not supported while the library is
 * loaded. */
#ifndef BARACUDA_U8_RRR_NOALLOC_SCRATCH_BYTES
#define BARACUDA_U8_RRR_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
#endif
int32_t baracuda_kernels_gemm_u8_rrr_gfx950_noalloc_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta, void *stream);
#define BK_U8_RRR_BIAS_DECL(EPI, BIAS)                                                          \
    int32_t baracuda_kernels_gemm_u8_rrr_gfx950_##EPI##_##BIAS##_run(                           \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha,         \
        float beta, void *workspace, size_t workspace_bytes, void *stream);                      \
    int32_t baracuda_kernels_gemm_u8_rrr_gfx950_##EPI##_##BIAS##_can_implement(                 \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb, \
        const void *c, int64_t ldc, const void *d, int64_t ldd);
BK_U8_RRR_BIAS_DECL(bias, f32)
BK_U8_RRR_BIAS_DECL(bias_relu, f32)
BK_U8_RRR_BIAS_DECL(bias_gelu, f32)
BK_U8_RRR_BIAS_DECL(bias_silu, f32)
BK_U8_RRR_BIAS_DECL(bias, i32)
BK_U8_RRR_BIAS_DECL(bias_relu, i32)
BK_U8_RRR_BIAS_DECL(bias_gelu, i32)
BK_U8_RRR_BIAS_DECL(bias_silu, i32)
#undef BK_U8_RRR_BIAS_DECL

/* ======================= MoE grouped GEMM, bf16 / f16 (reference ABI) =====
 * Same names and ABI as baracuda_kernels_moe_wmma_{f16,bf16}_{run,can_implement}
 * (crates/baracuda-kernels-sys/kernels/moe/moe_wmma.cu:121-209): input
 * [*, size_k], weights [num_experts, size_n, size_k] in the element type,
 * f32 accumulation, out[sorted_token_ids[p], n] = T(acc [* topk_weights[...]]).
 * expert_counts / expert_offsets are filled here; is_prefill is a hint. */
#define BK_MOE_WMMA_DECL(TAG)                                                                   \
    int32_t baracuda_kernels_moe_wmma_##TAG##_run(                                              \
        const void *input, const void *weights, const int32_t *sorted_token_ids,                \
        const int32_t *expert_ids, const float *topk_weights, void *output,                     \
        int32_t *expert_counts, int32_t *expert_offsets, int32_t num_experts, int32_t topk,     \
        int32_t size_m, int32_t size_n, int32_t size_k, int32_t is_prefill, void *workspace,    \
        size_t workspace_bytes, void *stream);                                                  \
    int32_t baracuda_kernels_moe_wmma_##TAG##_can_implement(int32_t num_experts, int32_t topk, \
                                                            int32_t size_m, int32_t size_n,    \
                                                            int32_t size_k, int32_t is_prefill);
BK_MOE_WMMA_DECL(bf16)
BK_MOE_WMMA_DECL(f16)
#undef BK_MOE_WMMA_DECL

/* ======================= FP8 delayed-scaling quantizer ===================
 * Same ABI as crates/baracuda-transformer-engine-sys/csrc/baracuda_te_shim.cu
 * (bound in crates/baracuda-transformer-engine-sys/src/lib.rs:95-257).
 * Status 0 ok, 1 invalid argument, 5 launch failure.  fmt 0 = e4m3, 1 = e5m2;
 * dtype 0 = f32, 1 = f16, 2 = bf16. */
int32_t baracuda_te_fp8_format_e4m3(void);
int32_t baracuda_te_fp8_format_e5m2(void);
float baracuda_te_fp8_max_representable(int32_t fmt);
/* out[i] = sat_fp8(x[i] * scale[0]); amax_history[write_pos] = max(., max|x|) */
int32_t baracuda_te_fused_cast_amax_run(const void *x_in, void *x_out, const float *scale,
                                        float *amax_history, int32_t write_pos, int64_t numel,
                                        int32_t fmt, int32_t in_dtype, void *stream);
int32_t baracuda_te_fused_cast_amax_can_implement(const void *x_in, const void *x_out,
                                                  const float *scale, const float *amax_history,
                                                  int32_t write_pos, int64_t numel, int32_t fmt,
                                                  int32_t in_dtype);
/* y[i] = dec(x[i]) * scale_inv[0] */
int32_t baracuda_te_dequant_run(const void *x_in, void *y_out, const float *scale_inv, int64_t numel,
                                int32_t fmt, int32_t out_dtype, void *stream);
int32_t baracuda_te_dequant_can_implement(const void *x_in, const void *y_out, const float *scale_inv,
                                          int64_t numel, int32_t fmt, int32_t out_dtype);
/* scale = max_repr / max(history) (0 -> 1, inf -> max_repr), scale_inv = 1/that;
 * history[write_pos] = 0 */
int32_t baracuda_te_recipe_update_run(float *amax_history, float *scale, float *scale_inv,
                                      int32_t hist_len, int32_t write_pos, int32_t fmt, void *stream);
int32_t baracuda_te_recipe_update_can_implement(const float *amax_history, const float *scale,
                                                const float *scale_inv, int32_t hist_len,
                                                int32_t write_pos, int32_t fmt);
int32_t baracuda_te_recipe_init_run(float *amax_history, float *scale, float *scale_inv,
                                    int32_t hist_len, void *stream);
int32_t baracuda_te_recipe_init_can_implement(const float *amax_history, const float *scale,
                                              const float *scale_inv, int32_t hist_len);

/* ======================= embedding forward ===============================
 * out[n,:] = weight[idx[n],:], zero row when idx[n] == padding_idx, < 0 or
 * >= V; idx i32 (embedding_<T>) or i64 (embedding_i64idx_<T>), padding_idx
 * as i64 (INT32_MIN = none).  Same ABI as baracuda_kernels_embedding_*
 * (crates/baracuda-kernels-sys/kernels/include/baracuda_embedding.cuh:513-556,
 *  kernels/embedding/embedding.cu:7-15). */
#define BK_EMBED_DECL(NAME)                                                                     \
    int32_t baracuda_kernels_##NAME##_run(int64_t num_indices, int32_t num_embeddings,          \
                                          int32_t embedding_dim, int64_t padding_idx,           \
                                          const void *weight, const void *indices, void *out,   \
                                          void *workspace, size_t workspace_bytes, void *stream); \
    int32_t baracuda_kernels_##NAME##_can_implement(int64_t num_indices, int32_t num_embeddings, \
                                                    int32_t embedding_dim, int64_t padding_idx, \
                                                    const void *weight, const void *indices,    \
                                                    const void *out);
BK_EMBED_DECL(embedding_f32)
BK_EMBED_DECL(embedding_f64)
BK_EMBED_DECL(embedding_f16)
BK_EMBED_DECL(embedding_bf16)
BK_EMBED_DECL(embedding_i64idx_f32)
BK_EMBED_DECL(embedding_i64idx_f64)
BK_EMBED_DECL(embedding_i64idx_f16)
BK_EMBED_DECL(embedding_i64idx_bf16)
#undef BK_EMBED_DECL

/* ======================= per-token dynamic int8 quantization =============
 * Replaces baracuda_kernels_dynamic_range_quantize_per_token_sym_{f32,f64}_s8_{run,can_implement}
 * (crates/baracuda-kernels-sys/kernels/include/baracuda_quantize_compose.cuh:143-203,306-338,
 *  crates/baracuda-kernels-sys/kernels/quantize/compose.cu:19-22), same ABI:
 * scale[n] = max|x[n,:]| / qmax (1 for an all-zero row), q = clamp(rne(x * (1/scale)), qmin, qmax).
 * Accepts N > 65535 (the reference rejects it). */
#define BK_QUANT_DECL(TAG)                                                                       \
    int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_##TAG##_s8_run(               \
        int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, void *scale,        \
        void *output, void *workspace, size_t workspace_bytes, void *stream);                    \
    int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_##TAG##_s8_can_implement(      \
        int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, const void *scale,  \
        const void *output);
BK_QUANT_DECL(f32)
BK_QUANT_DECL(f64)
#undef BK_QUANT_DECL

/* New SKU (same family): bf16 activations in, f32 per-token scales out. */
int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_run(
    int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, void *scale,
    void *output, void *workspace, size_t workspace_bytes, void *stream);
int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_can_implement(
    int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, const void *scale,
    const void *output);

/* ======================= FP8 e4m3 GEMM, RCR layout ======================
 * OCP e4m3 (e4m3fn) operands, f32 accumulator. */

/* Replaces baracuda_kernels_gemm_fp8_e4m3_rcr_sm89_{run,workspace_size,can_implement}
 * (crates/baracuda-kernels-sys/kernels/gemm/gemm_fp8_e4m3_rcr_sm89.cu:31-67):
 * D = sat_e4m3(rne(alpha*acc + beta*dequant(C))). */
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, const void *d, int64_t ldd);

/* New SKU: per-tensor scales, bf16 out: D = bf16_rne((scale_a*scale_b) * acc). */
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    float scale_a, float scale_b, void *d, int64_t ldd,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd);

/* New SKU: f32 out, D = alpha * acc (exposes the f32 accumulator). */
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    float alpha, void *d, int64_t ldd, void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_workspace_size(int32_t m, int32_t n, int32_t k);
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd);

/* ======================= m = 1 decode GEMV ===============================*/

/* Replaces baracuda_kernels_gemv_dense_m1_{f32,f16,bf16}_{run,can_implement,workspace_size}
 * (crates/baracuda-kernels-sys/kernels/gemm/gemv_dense.cu:235-342), same ABI:
 * D[g,0,:] = alpha*A[g,0,:]·B[g] + beta*D[g,0,:], RRR (layout 0), f32 accumulate,
 * stride_b == 0 broadcasts B, beta == 0 never reads D.  The reference's
 * _workspace_size returns 0; here it returns batch * ceil(K/R) * N * 4
 * bytes (R = 16 rows for f16 / bf16, 8 for f32) for K >= 256, N * K >= 2^20
 * and N a multiple of 16 bytes of elements (0 otherwise): given that
 * workspace (16-byte aligned), _run reads B in contiguous row spans and sums
 * per-R-row partials in a fixed order (split-K, two launches); given none it
 * runs the column-segment kernel. */
#define BK_GEMV_DENSE_DECL(TAG)                                                                  \
    int32_t baracuda_kernels_gemv_dense_m1_##TAG##_run(                                          \
        int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout, float alpha, float beta, \
        const void *a, int64_t lda, int64_t stride_a, const void *b, int64_t ldb,                \
        int64_t stride_b, void *d, int64_t ldd, int64_t stride_d, void *workspace,               \
        size_t workspace_bytes, void *stream);                                                   \
    int32_t baracuda_kernels_gemv_dense_m1_##TAG##_can_implement(                                \
        int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout, int64_t lda,             \
        int64_t ldb, int64_t ldd, int64_t stride_a, int64_t stride_b, int64_t stride_d);        \
    size_t baracuda_kernels_gemv_dense_m1_##TAG##_workspace_size(                                \
        int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout);
BK_GEMV_DENSE_DECL(f32)
BK_GEMV_DENSE_DECL(f16)
BK_GEMV_DENSE_DECL(bf16)
#undef BK_GEMV_DENSE_DECL

/* New SKU (gemv_dense_m1 family): int8 weight-only decode GEMV,
 * d[n] = bf16_rne(scale[n] * sum_k x[k]*w[n,k]), w [N,K] int8 (ldw), x bf16 [K],
 * scale f32 [N], f32 accumulate in a fixed order (bit-identical replays). */
int32_t baracuda_kernels_gemv_s8w_m1_bf16_gfx950_run(
    int32_t n, int32_t k, const void *x, const void *w, int64_t ldw, const void *scale, void *d,
    void *workspace, size_t workspace_bytes, void *stream);
size_t baracuda_kernels_gemv_s8w_m1_bf16_gfx950_workspace_size(int32_t n, int32_t k);
int32_t baracuda_kernels_gemv_s8w_m1_bf16_gfx950_can_implement(int32_t n, int32_t k, int64_t ldw);

/* ======================= gather_rows =====================================
 * Replaces baracuda_kernels_gather_rows_{f16,bf16,f32}_{run,can_implement,workspace_size}
 * (crates/baracuda-kernels-sys/kernels/indexing/gather_rows.cu:122-148), same ABI:
 * dest[r,:] = table[idx[r],:], idx u32, idx >= V writes zeros. */
#define BK_GATHER_DECL(TAG)                                                                      \
    int32_t baracuda_kernels_gather_rows_##TAG##_run(void *dest, const void *table,              \
                                                     const void *idx, int64_t V, int64_t H,      \
                                                     int64_t n, void *stream);                   \
    int32_t baracuda_kernels_gather_rows_##TAG##_can_implement(int64_t V, int64_t H, int64_t n); \
    size_t baracuda_kernels_gather_rows_##TAG##_workspace_size(int64_t V, int64_t H, int64_t n);
BK_GATHER_DECL(f16)
BK_GATHER_DECL(bf16)
BK_GATHER_DECL(f32)
#undef BK_GATHER_DECL

/* ======================= grouped MoE int8 GEMM ===========================
 * New SKU in the moe_wmma family; argument order of
 * baracuda_kernels_moe_wmma_bf16_run (crates/baracuda-kernels-sys/kernels/moe/moe_wmma.cu:154-175)
 * plus scale_a (one f32 per input row) and scale_w [E*N].  Routing: pairs grouped by expert
 * through sorted_token_ids / expert_ids; input row = id / topk (id when
 * topk_weights != NULL); output row = id; expert_counts [E] and
 * expert_offsets [E+1] are caller buffers filled by the call.
 * out[id,n] = bf16_rne(((scale_a[in_row]*scale_w[e*N+n]) * acc) [* topk_weights[id]]).
 * Each of the two products is rounded to f32 in that order. */
int32_t baracuda_kernels_moe_s8_grouped_bf16_gfx950_run(
    const void *input, const void *weights, const int32_t *sorted_token_ids,
    const int32_t *expert_ids, const float *topk_weights, void *output,
    int32_t *expert_counts, int32_t *expert_offsets, int32_t num_experts, int32_t topk,
    int32_t size_m, int32_t size_n, int32_t size_k, const float *scale_a, const float *scale_w,
    void *workspace, size_t workspace_bytes, void *stream);
int32_t baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement(
    int32_t num_experts, int32_t topk, int32_t size_m, int32_t size_n, int32_t size_k);
size_t baracuda_kernels_moe_s8_grouped_bf16_gfx950_workspace_size(
    int32_t num_experts, int32_t topk, int32_t size_m, int32_t size_n, int32_t size_k);

/* int32-accumulator form of the grouped int8 MoE (no counterpart in the
 * reference, which has no int8 MoE; for callers that dequantize themselves
 * and for whole-output exact checks): the bf16 SKU's routing and kernel with
 * out[id, n] = acc as int32 [size_m, N]; input row = id / topk (no
 * topk_weights, no scales).  Workspace 0. */
int32_t baracuda_kernels_moe_s8_grouped_i32_gfx950_run(
    const void *input, const void *weights, const int32_t *sorted_token_ids,
    const int32_t *expert_ids, void *output, int32_t *expert_counts, int32_t *expert_offsets,
    int32_t num_experts, int32_t topk, int32_t size_m, int32_t size_n, int32_t size_k, void *stream);
int32_t baracuda_kernels_moe_s8_grouped_i32_gfx950_can_implement(
    int32_t num_experts, int32_t topk, int32_t size_m, int32_t size_n, int32_t size_k);

#ifdef __cplusplus
}
#endif

#endif /* BARACUDA_KERNELS_GFX950_H */
