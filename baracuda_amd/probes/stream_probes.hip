// stream_probes.hip -- measurement kernels, not product: read-only streaming
// probes over an int8 [N, 4096] matrix in the launch shapes an m=1 GEMV can
// take, to bound what the GEMV (gemv_s8w_m1_kernel) can reach on the same
// bytes.  Built into libbaracuda_probes.so; used by bench.py only.
#include <hip/hip_runtime.h>
#include <cstdint>

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int K = 4096;

__device__ __forceinline__ v4i ld(const int8_t *p, bool nt) {
    return nt ? __builtin_nontemporal_load(reinterpret_cast<const v4i *>(p)) : *reinterpret_cast<const v4i *>(p);
}

// ROWS rows per wave, WPG waves per workgroup, all of a wave's loads issued
// before the first use; STORE: one 4-byte store per wave (what a GEMV must
// write), else a store that never executes.
template <int ROWS, int WPG, bool NT, bool STORE>
__global__ __launch_bounds__(64 * WPG) void probe_kernel(int N, const int8_t *__restrict__ w,
                                                         uint32_t *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int wv = blockIdx.x * WPG + (threadIdx.x >> 6);
    const int row0 = wv * ROWS;
    if (row0 >= N) return;
    v4i v[4][ROWS];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) v[u][r] = ld(w + (int64_t)(row0 + r) * K + u * 1024 + lane * 16, NT);
    int acc = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc ^= v[u][r][0] ^ v[u][r][1] ^ v[u][r][2] ^ v[u][r][3];
    if (STORE) {
        // every lane's value feeds the stored word, so no lane's loads are dropped
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
        if (lane == 63) out[wv] = (uint32_t)acc;
    } else if (acc == 0x12345678) {
        out[wv] = (uint32_t)acc;
    }
}

// Persistent: gridDim.x * WPG waves, wave v reads row pairs v, v + V, ...
// with the next pair's loads issued before the current pair is consumed.
__device__ __forceinline__ void ld_pair(v4i (&b)[4][2], const int8_t *w, int pr, int lane) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < 2; ++r) b[u][r] = ld(w + (int64_t)(2 * pr + r) * K + u * 1024 + lane * 16, true);
}

__global__ __launch_bounds__(64) void probe_persistent_kernel(int N, const int8_t *__restrict__ w,
                                                               uint32_t *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int V = gridDim.x, NP = N / 2;
    int p0 = blockIdx.x;
    if (p0 >= NP) return;
    v4i A[4][2], B[4][2];
    int acc = 0;
    ld_pair(A, w, p0, lane);
    while (true) {
        const int p1 = p0 + V;
        ld_pair(B, w, min(p1, NP - 1), lane);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < 2; ++r) acc ^= A[u][r][0] ^ A[u][r][1] ^ A[u][r][2] ^ A[u][r][3];
        if (p1 >= NP) break;
        const int p2 = p1 + V;
        ld_pair(A, w, min(p2, NP - 1), lane);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < 2; ++r) acc ^= B[u][r][0] ^ B[u][r][1] ^ B[u][r][2] ^ B[u][r][3];
        if (p2 >= NP) break;
        p0 = p2;
    }
    if (acc == 0x12345678) out[blockIdx.x] = (uint32_t)acc;
}

}  // namespace

extern "C" {

// Probe names, in the order of baracuda_probe_run's `kind`.
const char *baracuda_probe_name(int kind) {
    static const char *names[] = {
        "read_2rows_per_wave_nt",   "read_1row_per_wave_nt",     "read_4rows_per_wave_nt",
        "read_2rows_4wave_groups_nt", "read_2rows_per_wave_plain", "read_persistent_1024_waves",
        "read_persistent_2048_waves", "read_persistent_3584_waves", "read_2rows_per_wave_nt_plus_store"};
    return kind >= 0 && kind < 9 ? names[kind] : nullptr;
}

// One probe launch over w [N, 4096] int8 (N even); `out` holds N / 2 words.
// Returns 0, or 1 for an unknown kind / shape.
int32_t baracuda_probe_run(int32_t kind, const void *w, int32_t n, void *out, void *stream) {
    if (n <= 0 || n % 4 != 0) return 1;
    const int8_t *wp = static_cast<const int8_t *>(w);
    uint32_t *o = static_cast<uint32_t *>(out);
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (kind) {
    case 0: hipLaunchKernelGGL((probe_kernel<2, 1, true, false>), dim3(n / 2), dim3(64), 0, s, n, wp, o); break;
    case 1: hipLaunchKernelGGL((probe_kernel<1, 1, true, false>), dim3(n), dim3(64), 0, s, n, wp, o); break;
    case 2: hipLaunchKernelGGL((probe_kernel<4, 1, true, false>), dim3(n / 4), dim3(64), 0, s, n, wp, o); break;
    case 3: hipLaunchKernelGGL((probe_kernel<2, 4, true, false>), dim3((n / 2 + 3) / 4), dim3(256), 0, s, n, wp, o); break;
    case 4: hipLaunchKernelGGL((probe_kernel<2, 1, false, false>), dim3(n / 2), dim3(64), 0, s, n, wp, o); break;
    case 5: hipLaunchKernelGGL(probe_persistent_kernel, dim3(1024), dim3(64), 0, s, n, wp, o); break;
    case 6: hipLaunchKernelGGL(probe_persistent_kernel, dim3(2048), dim3(64), 0, s, n, wp, o); break;
    case 7: hipLaunchKernelGGL(probe_persistent_kernel, dim3(3584), dim3(64), 0, s, n, wp, o); break;
    case 8: hipLaunchKernelGGL((probe_kernel<2, 1, true, true>), dim3(n / 2), dim3(64), 0, s, n, wp, o); break;
    default: return 1;
    }
    return hipPeekAtLastError() == hipSuccess ? 0 : 1;
}

}  // extern "C"
