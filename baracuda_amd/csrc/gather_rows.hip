// gather_rows.hip -- capture-safe row gather for gfx950.
//
//   dest[r, :] = table[idx[r], :]    (idx u32; idx >= V writes zeros)
//
// Same contract and C ABI as the reference
// (crates/baracuda-kernels-sys/kernels/indexing/gather_rows.cu:60-148):
// every output element is written exactly once by a plain store, all
// metadata is passed by value, no memset / atomics / allocation, so a
// captured graph replays bit-identically.
//
// MI355X layout: the copy moves 16-byte units (global_load/store_dwordx4),
// one unit per lane, grid-stride over n * row_units with a strict bound.  The
// index load is per lane but hits the same cache line for a whole row.
// Rows whose byte length is not a multiple of 16 (or misaligned buffers) use
// an element-wise variant of the same loop.
#include "bk_common.hpp"

namespace bk {
namespace {

__global__ __launch_bounds__(256) void gather_rows_v16_kernel(v4i *__restrict__ dest,
                                                            const v4i *__restrict__ table,
                                                            const uint32_t *__restrict__ idx,
                                                            int64_t V, int64_t units_per_row,
                                                            int64_t total_units) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < total_units; u += step) {
        const int64_t row = u / units_per_row;
        const int64_t col = u - row * units_per_row;
        const uint32_t v = idx[row];
        v4i val = {0, 0, 0, 0};
        if ((int64_t)v < V) val = table[(int64_t)v * units_per_row + col];
        dest[u] = val;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void gather_rows_elem_kernel(T *__restrict__ dest,
                                                             const T *__restrict__ table,
                                                             const uint32_t *__restrict__ idx,
                                                             int64_t V, int64_t H, int64_t total) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
        const int64_t row = e / H;
        const int64_t col = e - row * H;
        const uint32_t v = idx[row];
        dest[e] = ((int64_t)v < V) ? table[(int64_t)v * H + col] : (T)0;
    }
}

template <typename T>
int32_t launch_gather(void *dest, const void *table, const void *idx, int64_t V, int64_t H,
                      int64_t n, hipStream_t stream) {
    if (V <= 0 || H <= 0 || n < 0) return kInvalid;
    if (n == 0) return kOk;
    if (!dest || !table || !idx) return kInvalid;
    constexpr int kBlock = 256;
    constexpr int64_t kMaxBlocks = 65535;
    const int64_t row_bytes = H * (int64_t)sizeof(T);
    const bool vec = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(dest) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(table) & 15u) == 0;
    if (vec) {
        const int64_t upr = row_bytes / 16;
        const int64_t total = n * upr;
        int64_t blocks = (total + kBlock - 1) / kBlock;
        blocks = blocks > kMaxBlocks ? kMaxBlocks : blocks;
        hipLaunchKernelGGL(gather_rows_v16_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, stream,
                           (v4i *)dest, (const v4i *)table, (const uint32_t *)idx, V, upr, total);
    } else {
        const int64_t total = n * H;
        int64_t blocks = (total + kBlock - 1) / kBlock;
        blocks = blocks > kMaxBlocks ? kMaxBlocks : blocks;
        hipLaunchKernelGGL((gather_rows_elem_kernel<T>), dim3((unsigned)blocks), dim3(kBlock), 0,
                           stream, (T *)dest, (const T *)table, (const uint32_t *)idx, V, H, total);
    }
    return launch_status();
}

}  // namespace
}  // namespace bk

using namespace bk;

#define BK_GATHER_ROWS(TAG, TY)                                                                  \
    extern "C" int32_t baracuda_kernels_gather_rows_##TAG##_run(                                 \
        void *dest, const void *table, const void *idx, int64_t V, int64_t H, int64_t n,         \
        void *stream) {                                                                          \
        return launch_gather<TY>(dest, table, idx, V, H, n, (hipStream_t)stream);               \
    }                                                                                            \
    extern "C" int32_t baracuda_kernels_gather_rows_##TAG##_can_implement(int64_t V, int64_t H,  \
                                                                          int64_t n) {           \
        if (V <= 0 || H <= 0 || n < 0) return kInvalid;                                          \
        return kOk;                                                                              \
    }                                                                                            \
    extern "C" size_t baracuda_kernels_gather_rows_##TAG##_workspace_size(int64_t V, int64_t H,  \
                                                                          int64_t n) {           \
        (void)V; (void)H; (void)n;                                                               \
        return 0;                                                                                \
    }

BK_GATHER_ROWS(f16, uint16_t)
BK_GATHER_ROWS(bf16, uint16_t)
BK_GATHER_ROWS(f32, uint32_t)

#undef BK_GATHER_ROWS
