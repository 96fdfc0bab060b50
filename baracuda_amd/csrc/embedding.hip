// embedding.hip -- embedding forward (row lookup with padding_idx) for gfx950.
//
// Semantics of embedding_kernel / launch_embedding
// (crates/baracuda-kernels-sys/kernels/include/baracuda_embedding.cuh:61-115):
//   out[n, :] = weight[idx[n], :]
//   out[n, :] = 0  when idx[n] == padding_idx, idx[n] < 0 or idx[n] >= V
// with idx i32 or i64 and padding_idx passed as i64 (INT32_MIN = disabled).
// Pure copy: bit-exact for every element type.
//
// MI355X layout: a 2-D grid, rows on y (grid-strided past 65535), 16-byte
// units of a row on x, so each row's index is read and tested once per
// thread and no thread divides by the row length.  Rows whose byte length
// or bases are not 16-byte aligned fall back to one element per lane with
// the same row mapping.
#include "bk_common.hpp"

namespace bk {
namespace {

template <typename Unit, typename IndexT>
__global__ __launch_bounds__(256) void embedding_rows_kernel(Unit *__restrict__ out,
                                                             const Unit *__restrict__ weight,
                                                             const IndexT *__restrict__ idx,
                                                             int64_t n, int32_t V,
                                                             int64_t row_units, int64_t padding_idx) {
    const int64_t u0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t ustep = (int64_t)gridDim.x * blockDim.x;
    for (int64_t row = blockIdx.y; row < n; row += gridDim.y) {
        const int64_t v = (int64_t)idx[row];
        const bool zero = v == padding_idx || v < 0 || v >= (int64_t)V;
        Unit *dst = out + row * row_units;
        if (zero) {
            for (int64_t u = u0; u < row_units; u += ustep) dst[u] = Unit{};
        } else {
            const Unit *src = weight + v * row_units;
            for (int64_t u = u0; u < row_units; u += ustep) dst[u] = src[u];
        }
    }
}

template <typename T, typename IndexT>
int32_t launch_embedding(int64_t num_indices, int32_t V, int32_t D, int64_t padding_idx,
                         const void *weight, const void *indices, void *out, hipStream_t stream) {
    if (num_indices < 0 || V < 0 || D < 0) return kInvalid;
    if (num_indices == 0 || D == 0) return kOk;
    constexpr int kBlock = 256;
    const int64_t row_bytes = (int64_t)D * (int64_t)sizeof(T);
    const bool vec = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(weight) & 15u) == 0;
    const int64_t units = vec ? row_bytes / 16 : (int64_t)D;
    int64_t gx = (units + kBlock - 1) / kBlock;
    gx = gx > 1024 ? 1024 : gx;
    const int64_t gy = num_indices > 65535 ? 65535 : num_indices;
    const dim3 grid((unsigned)gx, (unsigned)gy);
    if (vec)
        hipLaunchKernelGGL((embedding_rows_kernel<v4i, IndexT>), grid, dim3(kBlock), 0, stream,
                           (v4i *)out, (const v4i *)weight, (const IndexT *)indices, num_indices, V,
                           units, padding_idx);
    else
        hipLaunchKernelGGL((embedding_rows_kernel<T, IndexT>), grid, dim3(kBlock), 0, stream,
                           (T *)out, (const T *)weight, (const IndexT *)indices, num_indices, V,
                           units, padding_idx);
    return launch_status();
}

struct Half16 { uint16_t bits; };   // f16 / bf16 element: a 2-byte copy

}  // namespace
}  // namespace bk

using namespace bk;

extern "C" {

// Same ABI as baracuda_kernels_embedding[_i64idx]_{f32,f64,f16,bf16}_{run,can_implement}
// (baracuda_embedding.cuh:513-556 macro, kernels/embedding/embedding.cu:7-15).
#define BK_EMBEDDING(NAME, T, IDX)                                                                 \
    int32_t baracuda_kernels_##NAME##_run(int64_t num_indices, int32_t num_embeddings,            \
                                          int32_t embedding_dim, int64_t padding_idx,             \
                                          const void *weight, const void *indices, void *out,     \
                                          void *workspace, size_t workspace_bytes, void *stream) { \
        (void)workspace; (void)workspace_bytes;                                                    \
        if (num_indices < 0) return kInvalid;                                                      \
        if (num_indices == 0) return kOk;                                                          \
        if (!weight || !indices || !out) return kInvalid;                                          \
        return launch_embedding<T, IDX>(num_indices, num_embeddings, embedding_dim, padding_idx,   \
                                        weight, indices, out, (hipStream_t)stream);                \
    }                                                                                              \
    int32_t baracuda_kernels_##NAME##_can_implement(int64_t num_indices, int32_t num_embeddings,  \
                                                    int32_t embedding_dim, int64_t padding_idx,   \
                                                    const void *weight, const void *indices,      \
                                                    const void *out) {                            \
        (void)padding_idx; (void)weight; (void)indices; (void)out;                                 \
        if (num_indices < 0 || num_embeddings < 0 || embedding_dim < 0) return kInvalid;           \
        return kOk;                                                                                \
    }

BK_EMBEDDING(embedding_f32, float, int32_t)
BK_EMBEDDING(embedding_f64, double, int32_t)
BK_EMBEDDING(embedding_f16, Half16, int32_t)
BK_EMBEDDING(embedding_bf16, Half16, int32_t)
BK_EMBEDDING(embedding_i64idx_f32, float, int64_t)
BK_EMBEDDING(embedding_i64idx_f64, double, int64_t)
BK_EMBEDDING(embedding_i64idx_f16, Half16, int64_t)
BK_EMBEDDING(embedding_i64idx_bf16, Half16, int64_t)
#undef BK_EMBEDDING

}  // extern "C"
