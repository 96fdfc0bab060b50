// te_fp8.hip -- TransformerEngine-style FP8 delayed-scaling quantizer for
// gfx950: the producer of the FP8 GEMM operands.
//
// Same C ABI and semantics as crates/baracuda-transformer-engine-sys/csrc/
// baracuda_te_shim.cu (status 0 ok, 1 invalid argument, 5 launch failure):
//   fused_cast_amax  out[i] = sat_fp8(x[i] * scale[0]);  amax_history[write_pos]
//                    = max(itself, max_i |x[i]|)   (NaN inputs ignored by the max)
//   dequant          y[i] = dec(x[i]) * scale_inv[0]  (f32 / f16 / bf16 out, RNE)
//   recipe_update    amax = max(history) (0 -> 1, non-finite -> max_repr);
//                    scale = max_repr / amax, scale_inv = amax / max_repr;
//                    history[write_pos] = 0
//   recipe_init      scale = scale_inv = 1, history = 0
// Input / output dtype tags 0 = f32, 1 = f16, 2 = bf16; fp8 format 0 = e4m3,
// 1 = e5m2.
//
// MI355X layout: the cast and dequant are HBM-bound streams; each thread
// moves 2 (cast) or 4 (dequant) units of 8 elements per step (16-byte, or
// 2 x 16-byte for f32, loads, all issued before the first conversion, and
// 8-byte fp8 stores), grid-strided over at most 2048 workgroups.  The amax
// is reduced across the wave with shuffles, across the workgroup in LDS,
// and folded into the history slot with an integer atomicMax on the bits
// of a non-negative float (order-preserving), issued only by workgroups
// whose max exceeds the slot's current value.  Init is
// a kernel rather than host copies, so it can be captured in a graph.
#include "bk_common.hpp"

namespace bk {
namespace {

constexpr int kTeBlock = 256;
constexpr int kTeMaxHistory = 8192;
constexpr int kTeMaxGrid = 2048;
constexpr int kTeUnroll = 4;       // dequant: 8-element units per thread per step
constexpr int kTeCastUnroll = 2;   // cast
enum TeStatus : int32_t { kTeOk = 0, kTeInvalid = 1, kTeLaunch = 5 };

__host__ __device__ inline float te_max_repr(int32_t fmt) {
    return fmt == 0 ? 448.0f : (fmt == 1 ? 57344.0f : 1.0f);
}

struct F16 { uint16_t bits; };
struct BF16 { uint16_t bits; };

template <typename T> __device__ inline float te_ld(const T *p);
template <> __device__ inline float te_ld<float>(const float *p) { return *p; }
template <> __device__ inline float te_ld<F16>(const F16 *p) { return f16_to_f32(p->bits); }
template <> __device__ inline float te_ld<BF16>(const BF16 *p) { return bf16_to_f32(p->bits); }

template <typename T> __device__ inline void te_st(T *p, float v);
template <> __device__ inline void te_st<float>(float *p, float v) { *p = v; }
template <> __device__ inline void te_st<F16>(F16 *p, float v) { p->bits = f32_to_f16_rne(v); }
template <> __device__ inline void te_st<BF16>(BF16 *p, float v) { p->bits = f32_to_bf16_rne(v); }

// 8 consecutive inputs as floats (one 16-byte load for 2-byte types, two for f32).
template <typename T>
__device__ inline void te_ld8(const T *p, float (&v)[8]) {
    if constexpr (sizeof(T) == 4) {
        const v4f a = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p));
        const v4f b = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p + 4));
#pragma unroll
        for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
    } else {
        const v4i w = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(p));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = (uint32_t)w[i];
            v[2 * i] = te_ld<T>(reinterpret_cast<const T *>(&u));
            const uint16_t hi = (uint16_t)(u >> 16);
            v[2 * i + 1] = te_ld<T>(reinterpret_cast<const T *>(&hi));
        }
    }
}

__device__ inline float block_max_nonneg(float v, float *red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kTeBlock / 64; ++w) m = fmaxf(m, red[w]);
    return m;
}

// Vec: 16-byte aligned input and 8-byte aligned output (then 8-element steps;
// the numel % 8 tail is done element-wise by the first threads of block 0).
template <typename T, int FMT, bool Vec>
__global__ __launch_bounds__(kTeBlock) void te_cast_amax_kernel(const T *__restrict__ x,
                                                                 uint8_t *__restrict__ out,
                                                                 const float *__restrict__ scale,
                                                                 float *__restrict__ amax_slot,
                                                                 int64_t numel) {
    __shared__ float red[kTeBlock / 64];
    const float s = scale[0];
    float tmax = 0.0f;
    const int64_t tid = (int64_t)blockIdx.x * kTeBlock + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * kTeBlock;
    if constexpr (Vec) {
        // kTeUnroll independent 8-element units per thread per step, all
        // loads issued before any conversion: 4x the bytes in flight.
        const int64_t units = numel >> 3;
        for (int64_t u0 = tid; u0 < units; u0 += kTeCastUnroll * step) {
            float v[kTeCastUnroll][8];
#pragma unroll
            for (int j = 0; j < kTeCastUnroll; ++j) {
                const int64_t u = u0 + j * step;
                if (u < units) te_ld8<T>(x + 8 * u, v[j]);
            }
#pragma unroll
            for (int j = 0; j < kTeCastUnroll; ++j) {
                const int64_t u = u0 + j * step;
                if (u >= units) break;
                float y[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    tmax = fmaxf(tmax, fabsf(v[j][i]));
                    y[i] = v[j][i] * s;
                }
                const uint32_t lo = f32x4_to_fp8x4_satfinite<FMT>(y[0], y[1], y[2], y[3]);
                const uint32_t hi = f32x4_to_fp8x4_satfinite<FMT>(y[4], y[5], y[6], y[7]);
                __builtin_nontemporal_store(v2i{(int)lo, (int)hi}, reinterpret_cast<v2i *>(out + 8 * u));
            }
        }
        const int64_t t0 = units << 3;
        if (blockIdx.x == 0 && t0 + threadIdx.x < numel) {
            const float v = te_ld<T>(x + t0 + threadIdx.x);
            tmax = fmaxf(tmax, fabsf(v));
            out[t0 + threadIdx.x] = f32_to_fp8_satfinite<FMT>(v * s);
        }
    } else {
        for (int64_t i = tid; i < numel; i += step) {
            const float v = te_ld<T>(x + i);
            tmax = fmaxf(tmax, fabsf(v));
            out[i] = f32_to_fp8_satfinite<FMT>(v * s);
        }
    }
    // The slot only grows: a workgroup whose max does not exceed the value
    // it reads (possibly stale, i.e. lower) skips its atomic.  With one
    // atomic per workgroup on one address, the atomics serialise: 2048 of
    // them cost 38 us against 27 us with the check (14336 x 4096 bf16).
    const float m = block_max_nonneg(tmax, red);
    if (threadIdx.x == 0) {
        int *slot = reinterpret_cast<int *>(amax_slot);
        if (__float_as_int(m) > __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
            atomicMax(slot, __float_as_int(m));
    }
}

template <typename T, int FMT, bool Vec>
__global__ __launch_bounds__(kTeBlock) void te_dequant_kernel(const uint8_t *__restrict__ x,
                                                               T *__restrict__ y,
                                                               const float *__restrict__ scale_inv,
                                                               int64_t numel) {
    const float si = scale_inv[0];
    const int64_t tid = (int64_t)blockIdx.x * kTeBlock + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * kTeBlock;
    if constexpr (Vec) {
        const int64_t units = numel >> 3;
        for (int64_t u0 = tid; u0 < units; u0 += kTeUnroll * step) {
            v2i w[kTeUnroll];
#pragma unroll
            for (int j = 0; j < kTeUnroll; ++j) {
                const int64_t u = u0 + j * step;
                if (u < units) w[j] = *reinterpret_cast<const v2i *>(x + 8 * u);
            }
#pragma unroll
            for (int j = 0; j < kTeUnroll; ++j) {
                const int64_t u = u0 + j * step;
                if (u >= units) break;
                T o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint8_t b = (uint8_t)((uint32_t)w[j][i >> 2] >> (8 * (i & 3)));
                    te_st<T>(&o[i], fp8_to_f32<FMT>(b) * si);
                }
                if constexpr (sizeof(T) == 4) {
                    *reinterpret_cast<v4f *>(y + 8 * u) = *reinterpret_cast<const v4f *>(&o[0]);
                    *reinterpret_cast<v4f *>(y + 8 * u + 4) = *reinterpret_cast<const v4f *>(&o[4]);
                } else {
                    *reinterpret_cast<v4i *>(y + 8 * u) = *reinterpret_cast<const v4i *>(&o[0]);
                }
            }
        }
        const int64_t t0 = units << 3;
        if (blockIdx.x == 0 && t0 + threadIdx.x < numel)
            te_st<T>(y + t0 + threadIdx.x, fp8_to_f32<FMT>(x[t0 + threadIdx.x]) * si);
    } else {
        for (int64_t i = tid; i < numel; i += step) te_st<T>(y + i, fp8_to_f32<FMT>(x[i]) * si);
    }
}

__global__ __launch_bounds__(kTeBlock) void te_recipe_update_kernel(float *__restrict__ hist,
                                                                     float *__restrict__ scale,
                                                                     float *__restrict__ scale_inv,
                                                                     int32_t hist_len,
                                                                     int32_t write_pos,
                                                                     float max_repr) {
    __shared__ float red[kTeBlock / 64];
    float tmax = 0.0f;
    for (int i = threadIdx.x; i < hist_len; i += kTeBlock) {
        const float v = hist[i];
        tmax = v > tmax ? v : tmax;   // NaN entries never win, as in the reference
    }
    float amax = block_max_nonneg(tmax, red);
    if (threadIdx.x == 0) {
        if (!(amax > 0.0f)) amax = 1.0f;
        if (!__builtin_isfinite(amax)) amax = max_repr;
        scale[0] = max_repr / amax;
        scale_inv[0] = amax / max_repr;
        hist[write_pos] = 0.0f;
    }
}

__global__ __launch_bounds__(kTeBlock) void te_recipe_init_kernel(float *__restrict__ hist,
                                                                   float *__restrict__ scale,
                                                                   float *__restrict__ scale_inv,
                                                                   int32_t hist_len) {
    for (int i = threadIdx.x; i < hist_len; i += kTeBlock) hist[i] = 0.0f;
    if (threadIdx.x == 0) {
        scale[0] = 1.0f;
        scale_inv[0] = 1.0f;
    }
}

inline int te_grid(int64_t work) {
    const int64_t g = (work + kTeBlock - 1) / kTeBlock;
    return (int)(g < 1 ? 1 : (g > kTeMaxGrid ? kTeMaxGrid : g));
}

inline int32_t te_launch_status() { return hipGetLastError() == hipSuccess ? kTeOk : kTeLaunch; }

template <typename T, int FMT>
int32_t te_cast(const void *x, void *out, const float *scale, float *slot, int64_t numel,
                hipStream_t s) {
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & 7u) == 0;
    if (vec)
        hipLaunchKernelGGL((te_cast_amax_kernel<T, FMT, true>),
                           dim3(te_grid(((numel >> 3) + kTeCastUnroll - 1) / kTeCastUnroll)), dim3(kTeBlock),
                           0, s, (const T *)x, (uint8_t *)out, scale, slot, numel);
    else
        hipLaunchKernelGGL((te_cast_amax_kernel<T, FMT, false>), dim3(te_grid(numel)), dim3(kTeBlock), 0,
                           s, (const T *)x, (uint8_t *)out, scale, slot, numel);
    return te_launch_status();
}

template <typename T, int FMT>
int32_t te_dequant(const void *x, void *y, const float *scale_inv, int64_t numel, hipStream_t s) {
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 7u) == 0 &&
                     (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    if (vec)
        hipLaunchKernelGGL((te_dequant_kernel<T, FMT, true>), dim3(te_grid(((numel >> 3) + kTeUnroll - 1) / kTeUnroll)), dim3(kTeBlock), 0,
                           s, (const uint8_t *)x, (T *)y, scale_inv, numel);
    else
        hipLaunchKernelGGL((te_dequant_kernel<T, FMT, false>), dim3(te_grid(numel)), dim3(kTeBlock), 0, s,
                           (const uint8_t *)x, (T *)y, scale_inv, numel);
    return te_launch_status();
}

template <int FMT>
int32_t te_cast_dtype(int32_t dt, const void *x, void *out, const float *scale, float *slot,
                      int64_t numel, hipStream_t s) {
    if (dt == 0) return te_cast<float, FMT>(x, out, scale, slot, numel, s);
    if (dt == 1) return te_cast<F16, FMT>(x, out, scale, slot, numel, s);
    return te_cast<BF16, FMT>(x, out, scale, slot, numel, s);
}

template <int FMT>
int32_t te_dequant_dtype(int32_t dt, const void *x, void *y, const float *si, int64_t numel,
                         hipStream_t s) {
    if (dt == 0) return te_dequant<float, FMT>(x, y, si, numel, s);
    if (dt == 1) return te_dequant<F16, FMT>(x, y, si, numel, s);
    return te_dequant<BF16, FMT>(x, y, si, numel, s);
}

}  // namespace
}  // namespace bk

using namespace bk;

extern "C" {

int32_t baracuda_te_fp8_format_e4m3() { return 0; }
int32_t baracuda_te_fp8_format_e5m2() { return 1; }
float baracuda_te_fp8_max_representable(int32_t fmt) { return te_max_repr(fmt); }

int32_t baracuda_te_fused_cast_amax_can_implement(const void *x_in, const void *x_out,
                                                  const float *scale, const float *amax_history,
                                                  int32_t write_pos, int64_t numel, int32_t fmt,
                                                  int32_t in_dtype) {
    (void)x_in; (void)x_out; (void)scale; (void)amax_history;
    if (numel < 0 || write_pos < 0) return kTeInvalid;
    if (fmt != 0 && fmt != 1) return kTeInvalid;
    if (in_dtype < 0 || in_dtype > 2) return kTeInvalid;
    return kTeOk;
}

int32_t baracuda_te_fused_cast_amax_run(const void *x_in, void *x_out, const float *scale,
                                        float *amax_history, int32_t write_pos, int64_t numel,
                                        int32_t fmt, int32_t in_dtype, void *stream) {
    if (!x_in || !x_out || !scale || !amax_history) return kTeInvalid;
    if (numel <= 0 || write_pos < 0) return kTeInvalid;
    if (fmt != 0 && fmt != 1) return kTeInvalid;
    if (in_dtype < 0 || in_dtype > 2) return kTeInvalid;
    hipStream_t s = (hipStream_t)stream;
    float *slot = amax_history + write_pos;
    return fmt == 0 ? te_cast_dtype<FMT_E4M3>(in_dtype, x_in, x_out, scale, slot, numel, s)
                    : te_cast_dtype<FMT_E5M2>(in_dtype, x_in, x_out, scale, slot, numel, s);
}

int32_t baracuda_te_dequant_can_implement(const void *x_in, const void *y_out, const float *scale_inv,
                                          int64_t numel, int32_t fmt, int32_t out_dtype) {
    (void)x_in; (void)y_out; (void)scale_inv;
    if (numel < 0) return kTeInvalid;
    if (fmt != 0 && fmt != 1) return kTeInvalid;
    if (out_dtype < 0 || out_dtype > 2) return kTeInvalid;
    return kTeOk;
}

int32_t baracuda_te_dequant_run(const void *x_in, void *y_out, const float *scale_inv, int64_t numel,
                                int32_t fmt, int32_t out_dtype, void *stream) {
    if (!x_in || !y_out || !scale_inv) return kTeInvalid;
    if (numel <= 0) return kTeInvalid;
    if (fmt != 0 && fmt != 1) return kTeInvalid;
    if (out_dtype < 0 || out_dtype > 2) return kTeInvalid;
    hipStream_t s = (hipStream_t)stream;
    return fmt == 0 ? te_dequant_dtype<FMT_E4M3>(out_dtype, x_in, y_out, scale_inv, numel, s)
                    : te_dequant_dtype<FMT_E5M2>(out_dtype, x_in, y_out, scale_inv, numel, s);
}

int32_t baracuda_te_recipe_update_can_implement(const float *amax_history, const float *scale,
                                                const float *scale_inv, int32_t hist_len,
                                                int32_t write_pos, int32_t fmt) {
    (void)amax_history; (void)scale; (void)scale_inv;
    if (hist_len <= 0 || hist_len > kTeMaxHistory) return kTeInvalid;
    if (write_pos < 0 || write_pos >= hist_len) return kTeInvalid;
    if (fmt != 0 && fmt != 1) return kTeInvalid;
    return kTeOk;
}

int32_t baracuda_te_recipe_update_run(float *amax_history, float *scale, float *scale_inv,
                                      int32_t hist_len, int32_t write_pos, int32_t fmt, void *stream) {
    if (!amax_history || !scale || !scale_inv) return kTeInvalid;
    if (baracuda_te_recipe_update_can_implement(amax_history, scale, scale_inv, hist_len, write_pos,
                                                fmt) != kTeOk)
        return kTeInvalid;
    hipLaunchKernelGGL(te_recipe_update_kernel, dim3(1), dim3(kTeBlock), 0, (hipStream_t)stream,
                       amax_history, scale, scale_inv, hist_len, write_pos, te_max_repr(fmt));
    return te_launch_status();
}

int32_t baracuda_te_recipe_init_can_implement(const float *amax_history, const float *scale,
                                              const float *scale_inv, int32_t hist_len) {
    (void)amax_history; (void)scale; (void)scale_inv;
    if (hist_len <= 0 || hist_len > kTeMaxHistory) return kTeInvalid;
    return kTeOk;
}

int32_t baracuda_te_recipe_init_run(float *amax_history, float *scale, float *scale_inv,
                                    int32_t hist_len, void *stream) {
    if (!amax_history || !scale || !scale_inv) return kTeInvalid;
    if (hist_len <= 0 || hist_len > kTeMaxHistory) return kTeInvalid;
    hipLaunchKernelGGL(te_recipe_init_kernel, dim3(1), dim3(kTeBlock), 0, (hipStream_t)stream,
                       amax_history, scale, scale_inv, hist_len);
    return te_launch_status();
}

}  // extern "C"
