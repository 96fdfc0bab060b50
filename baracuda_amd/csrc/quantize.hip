// quantize.hip -- per-token symmetric dynamic-range int8 quantization for
// gfx950: the producer of the W8A8 GEMM's activation operand and its
// per-token scale.
//
// Semantics of dynamic_range_quantize_per_token_sym
// (crates/baracuda-kernels-sys/kernels/include/baracuda_quantize_compose.cuh:143-203):
//   max_abs  = max_d |x[n, d]|
//   scale[n] = max_abs > 0 ? max_abs / qmax : 1            (in the input type)
//   inv      = 1 / scale                                    (f32)
//   q[n, d]  = clamp(round_half_even(x[n, d] * inv), qmin, qmax)
// For the f64 input the reference evaluates in f32 after a narrowing load
// (qc_load_as_f32) and stores the scale back as f64; the same here.
//
// MI355X layout: one workgroup (256 threads) per row (grid-strided), the row
// is read once into registers with workgroup-coalesced loads (up to 64
// elements per thread, i.e. D <= 16384; bf16 rows as 16-byte chunks of 8),
// reduced with a wave butterfly + LDS, quantized from registers: one HBM read
// of x, one write of q (8-byte stores on the bf16 path).  Longer rows
// take a two-pass loop over global memory.  Max is exact
// in any order, so the result is bit-identical to the reference's.
#include "bk_common.hpp"

namespace bk {
namespace {

constexpr int kQBlock = 256;
constexpr int kQMaxPerThread = 64;   // register-resident row: D <= 256 * 64

// Load as f32 (qc_load_as_f32, baracuda_quantize_compose.cuh:69-89).
template <typename T> struct QIn;
template <> struct QIn<float> {
    __device__ static float ld(const float *p) { return *p; }
};
template <> struct QIn<double> {
    __device__ static float ld(const double *p) { return (float)*p; }
};
struct Bf16In { uint16_t bits; };   // element type: pointer steps of 2 bytes
template <> struct QIn<Bf16In> {
    __device__ static float ld(const Bf16In *p) { return bf16_to_f32(p->bits); }
};

__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kQBlock / 64; ++w) m = fmaxf(m, red[w]);
    return m;
}

// clamp(round_half_even(v * inv), qmin, qmax), the clamp in float before the
// conversion (rne_clamp: NaN -> 0, no out-of-range conversion).
__device__ __forceinline__ int8_t quant1(float v, float inv, float qmin, float qmax) {
    return (int8_t)(int)rne_clamp(v * inv, qmin, qmax);
}

// T: element type of x; S: type of the scale output.
template <typename T, typename S>
__global__ __launch_bounds__(kQBlock) void quantize_per_token_kernel(
    const T *__restrict__ x, S *__restrict__ scale, int8_t *__restrict__ q, int N, int D,
    int qmin, int qmax) {
    __shared__ float red[kQBlock / 64];
    const float fqmax = (float)qmax;
    const float fqmin = (float)qmin;
    for (int n = blockIdx.x; n < N; n += gridDim.x) {
        const T *row = x + (int64_t)n * D;
        int8_t *qrow = q + (int64_t)n * D;
        float vals[kQMaxPerThread];
        const bool resident = D <= kQBlock * kQMaxPerThread;
        float m = 0.0f;
        if (resident) {
            // element e = tid + kQBlock * i: coalesced across the workgroup.
#pragma unroll
            for (int i = 0; i < kQMaxPerThread; ++i) {
                const int e = threadIdx.x + kQBlock * i;
                vals[i] = e < D ? QIn<T>::ld(row + e) : 0.0f;
                m = fmaxf(m, fabsf(vals[i]));
            }
        } else {
            for (int e = threadIdx.x; e < D; e += kQBlock) m = fmaxf(m, fabsf(QIn<T>::ld(row + e)));
        }
        const float max_abs = block_max(m, red);
        const float s = max_abs > 0.0f ? max_abs / fqmax : 1.0f;
        const float inv = s != 0.0f ? 1.0f / s : 0.0f;
        if (threadIdx.x == 0) scale[n] = (S)s;
        if (resident) {
#pragma unroll
            for (int i = 0; i < kQMaxPerThread; ++i) {
                const int e = threadIdx.x + kQBlock * i;
                if (e < D) qrow[e] = quant1(vals[i], inv, fqmin, fqmax);
            }
        } else {
            for (int e = threadIdx.x; e < D; e += kQBlock)
                qrow[e] = quant1(QIn<T>::ld(row + e), inv, fqmin, fqmax);
        }
        __syncthreads();   // `red` is reused by the next row
    }
}

// Vector path for 2-byte inputs (bf16): 16-byte non-temporal loads of 8
// elements, 8-byte non-temporal int8 stores; chunk c = tid + kQBlock * i, kChunks chunks
// (8 * kChunks values) per thread held in registers (D <= 2048 * kChunks,
// D % 8 == 0, 16-byte aligned rows).  The launcher picks the smallest of
// 1, 2, 4, 8 chunks that holds the row: fewer registers keep more rows in
// flight (4096 x 4096: 14.3 us with 8 chunks, 10.9 us with 2).
template <typename S, int kChunks>
__global__ __launch_bounds__(kQBlock) void quantize_per_token_bf16v_kernel(
    const uint16_t *__restrict__ x, S *__restrict__ scale, int8_t *__restrict__ q, int N, int D,
    int qmin, int qmax) {
    __shared__ float red[kQBlock / 64];
    const float fqmax = (float)qmax;
    const float fqmin = (float)qmin;
    const int nch = D >> 3;
    for (int n = blockIdx.x; n < N; n += gridDim.x) {
        const v4i *row = reinterpret_cast<const v4i *>(x + (int64_t)n * D);
        v4i w[kChunks];
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int c = threadIdx.x + kQBlock * i;
            w[i] = c < nch ? __builtin_nontemporal_load(row + c) : v4i{0, 0, 0, 0};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint32_t u = (uint32_t)w[i][h];
                m = fmaxf(m, fabsf(__uint_as_float(u << 16)));
                m = fmaxf(m, fabsf(__uint_as_float(u & 0xffff0000u)));
            }
        }
        const float max_abs = block_max(m, red);
        const float s = max_abs > 0.0f ? max_abs / fqmax : 1.0f;
        const float inv = s != 0.0f ? 1.0f / s : 0.0f;
        if (threadIdx.x == 0) scale[n] = (S)s;
        int8_t *qrow = q + (int64_t)n * D;
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int c = threadIdx.x + kQBlock * i;
            if (c >= nch) break;
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint32_t u = (uint32_t)w[i][h];
                const uint32_t q0 = (uint8_t)quant1(__uint_as_float(u << 16), inv, fqmin, fqmax);
                const uint32_t q1 = (uint8_t)quant1(__uint_as_float(u & 0xffff0000u), inv, fqmin, fqmax);
                const uint32_t pair = q0 | (q1 << 8);
                if (h < 2) lo |= pair << (16 * h);
                else hi |= pair << (16 * (h - 2));
            }
            __builtin_nontemporal_store(v2i{(int)lo, (int)hi}, reinterpret_cast<v2i *>(qrow + 8 * c));
        }
        __syncthreads();   // `red` is reused by the next row
    }
}

// Rows of D <= 4096 bf16 values (D % 8 == 0, 16-byte aligned rows): one
// wave per row, four rows per workgroup, chunk c = lane + 64 i of the row
// in registers (kChunks <= 8), the max over a wave butterfly (no LDS, no
// barrier), 8-byte non-temporal int8 stores.  kEven: D == 512 kChunks, no
// per-chunk guards (they cost 0.7 us at 4096 x 4096).  4096 x 4096 over 24
// rotated input / output pairs: 10.05 us against 10.7-10.9 for
// quantize_per_token_bf16v_kernel and 9.45 us for a copy with the same
// loads and stores and no arithmetic (bit-identical).
constexpr int kQRowsPerBlock = 4;
template <typename S, int kChunks, bool kEven>
__global__ __launch_bounds__(64 * kQRowsPerBlock) void quantize_per_token_bf16w_kernel(
    const uint16_t *__restrict__ x, S *__restrict__ scale, int8_t *__restrict__ q, int N, int D,
    int qmin, int qmax) {
    const float fqmax = (float)qmax;
    const float fqmin = (float)qmin;
    const int nch = D >> 3, lane = threadIdx.x & 63;
    for (int n = blockIdx.x * kQRowsPerBlock + (threadIdx.x >> 6); n < N; n += gridDim.x * kQRowsPerBlock) {
        const v4i *row = reinterpret_cast<const v4i *>(x + (int64_t)n * D);
        v4i w[kChunks];
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int c = lane + 64 * i;
            w[i] = (kEven || c < nch) ? __builtin_nontemporal_load(row + c) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < kChunks; ++i)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint32_t u = (uint32_t)w[i][h];
                m = fmaxf(m, fabsf(__uint_as_float(u << 16)));
                m = fmaxf(m, fabsf(__uint_as_float(u & 0xffff0000u)));
            }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        const float s = m > 0.0f ? m / fqmax : 1.0f;
        const float inv = s != 0.0f ? 1.0f / s : 0.0f;
        if (lane == 0) scale[n] = (S)s;
        int8_t *qrow = q + (int64_t)n * D;
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int c = lane + 64 * i;
            if (!kEven && c >= nch) break;
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint32_t u = (uint32_t)w[i][h];
                const uint32_t q0 = (uint8_t)quant1(__uint_as_float(u << 16), inv, fqmin, fqmax);
                const uint32_t q1 = (uint8_t)quant1(__uint_as_float(u & 0xffff0000u), inv, fqmin, fqmax);
                const uint32_t pair = q0 | (q1 << 8);
                if (h < 2) lo |= pair << (16 * h);
                else hi |= pair << (16 * (h - 2));
            }
            __builtin_nontemporal_store(v2i{(int)lo, (int)hi}, reinterpret_cast<v2i *>(qrow + 8 * c));
        }
    }
}

int32_t quant_check(int32_t N, int32_t D, int32_t qmin, int32_t qmax) {
    if (N < 0 || D < 0) return kInvalid;
    if (qmin > qmax) return kInvalid;
    if (qmax <= 0) return kInvalid;
    return kOk;   // N > 65535 is accepted (rows are grid-strided)
}

template <typename T, typename S>
int32_t launch_quant(int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input,
                     void *scale, void *output, hipStream_t stream) {
    const int32_t st = quant_check(N, D, qmin, qmax);
    if (st != kOk) return st;
    if ((int64_t)N * D == 0) return kOk;
    if (!input || !scale || !output) return kInvalid;
    const int grid = N < 65535 ? N : 65535;
    if constexpr (sizeof(T) == 2) {
        const bool vec = D % 8 == 0 && D <= kQBlock * kQMaxPerThread &&
                         (reinterpret_cast<uintptr_t>(input) & 15u) == 0 &&
                         (reinterpret_cast<uintptr_t>(output) & 7u) == 0;
        if (vec) {
            const uint16_t *xi = (const uint16_t *)input;
            S *sc = (S *)scale;
            int8_t *qo = (int8_t *)output;
            const int nch = D / 8;
            if (nch <= 64 * 8) {
                const int wgrid = (N + kQRowsPerBlock - 1) / kQRowsPerBlock < 65535
                                      ? (N + kQRowsPerBlock - 1) / kQRowsPerBlock : 65535;
                const dim3 wb(64 * kQRowsPerBlock);
#define BK_QW(CH)                                                                                          \
    if (nch == 64 * (CH))                                                                                  \
        hipLaunchKernelGGL((quantize_per_token_bf16w_kernel<S, CH, true>), dim3(wgrid), wb, 0, stream, xi, \
                           sc, qo, N, D, qmin, qmax);                                                      \
    else                                                                                                   \
        hipLaunchKernelGGL((quantize_per_token_bf16w_kernel<S, CH, false>), dim3(wgrid), wb, 0, stream, xi, \
                           sc, qo, N, D, qmin, qmax);
                if (nch <= 64) { BK_QW(1) }
                else if (nch <= 128) { BK_QW(2) }
                else if (nch <= 256) { BK_QW(4) }
                else { BK_QW(8) }
#undef BK_QW
                return launch_status();
            }
            if (nch <= kQBlock)
                hipLaunchKernelGGL((quantize_per_token_bf16v_kernel<S, 1>), dim3(grid), dim3(kQBlock), 0, stream,
                                   xi, sc, qo, N, D, qmin, qmax);
            else if (nch <= 2 * kQBlock)
                hipLaunchKernelGGL((quantize_per_token_bf16v_kernel<S, 2>), dim3(grid), dim3(kQBlock), 0, stream,
                                   xi, sc, qo, N, D, qmin, qmax);
            else if (nch <= 4 * kQBlock)
                hipLaunchKernelGGL((quantize_per_token_bf16v_kernel<S, 4>), dim3(grid), dim3(kQBlock), 0, stream,
                                   xi, sc, qo, N, D, qmin, qmax);
            else
                hipLaunchKernelGGL((quantize_per_token_bf16v_kernel<S, 8>), dim3(grid), dim3(kQBlock), 0, stream,
                                   xi, sc, qo, N, D, qmin, qmax);
            return launch_status();
        }
    }
    hipLaunchKernelGGL((quantize_per_token_kernel<T, S>), dim3(grid), dim3(kQBlock), 0, stream,
                       (const T *)input, (S *)scale, (int8_t *)output, N, D, qmin, qmax);
    return launch_status();
}

}  // namespace
}  // namespace bk

using namespace bk;

extern "C" {

// Same ABI as baracuda_kernels_dynamic_range_quantize_per_token_sym_{f32,f64}_s8_*
// (baracuda_quantize_compose.cuh:306-338 macro, compose.cu:19-22).
#define BK_QUANT(TAG, TY)                                                                          \
    int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_##TAG##_s8_run(                  \
        int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, void *scale,          \
        void *output, void *workspace, size_t workspace_bytes, void *stream) {                     \
        (void)workspace; (void)workspace_bytes;                                                    \
        return launch_quant<TY, TY>(N, D, qmin, qmax, input, scale, output, (hipStream_t)stream);  \
    }                                                                                              \
    int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_##TAG##_s8_can_implement(        \
        int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, const void *scale,    \
        const void *output) {                                                                      \
        (void)input; (void)scale; (void)output;                                                    \
        return quant_check(N, D, qmin, qmax);                                                      \
    }

BK_QUANT(f32, float)
BK_QUANT(f64, double)
#undef BK_QUANT

// New SKU: bf16 activations in, f32 per-token scales out (what the W8A8 GEMM
// epilogue consumes), int8 out.
int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_run(
    int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, void *scale,
    void *output, void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    return launch_quant<Bf16In, float>(N, D, qmin, qmax, input, scale, output, (hipStream_t)stream);
}

int32_t baracuda_kernels_dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_can_implement(
    int32_t N, int32_t D, int32_t qmin, int32_t qmax, const void *input, const void *scale,
    const void *output) {
    (void)input; (void)scale; (void)output;
    return quant_check(N, D, qmin, qmax);
}

}  // extern "C"
