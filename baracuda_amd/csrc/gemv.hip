// gemv.hip -- capture-safe m=1 decode GEMVs for gfx950 (HBM-bound, no MFMA).
//
// 1. gemv_s8w_m1_bf16_gfx950 (new SKU): int8 weight-only decode GEMV
//      out[n] = bf16_rne( scale[n] * sum_k x[k] * w[n, k] ),  f32 accumulate
//    W is [N, K] int8 row-major (ldw), x bf16 [K], scale f32 [N], out bf16 [N].
//    One wave64 owns ROWS consecutive output rows; lane l reads the 16-byte
//    unit l of every 1 KiB K-chunk of each row (global_load_dwordx4, fully
//    coalesced 1 KiB per wave per row), keeps the matching 16 x values in
//    registers, and the 64 partial sums are folded by fixed DPP moves.
//    Per-lane order and reduction order are fixed, so every launch is
//    bit-identical (graph replay safe) and independent of the grid.
//
// 2. gemv_dense_m1_{f32,f16,bf16} (reference ABI,
//    crates/baracuda-kernels-sys/kernels/gemm/gemv_dense.cu:101-342):
//      D[g, j] = alpha * sum_k A[g, k] * B[g, k, j] + beta * D[g, j]   (RRR)
//    Workgroup of 1024 threads owns 64 columns; its 16 waves split K into
//    16 contiguous slices (lane = column, coalesced 64-wide row reads), and
//    the 16 partials are summed in LDS in slice order.  Fixed order => the
//    result does not depend on grid shape and replays bit-identically.
//    beta == 0 never reads D (write-only, gemv_dense.cu:163-169).
#include "bk_common.hpp"

namespace bk {
namespace {

// ---------------------------------------------------------------------------
// int8 weight-only GEMV
// ---------------------------------------------------------------------------
constexpr int kGemvWaves = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Wave total in lane 63 through DPP moves (no LDS round trips): pair and quad
// sums, half-row and row mirrors (16-lane sums), then row 15 -> row 1 / 3 and
// lane 31 -> rows 2, 3 broadcasts.  A fixed order, so every launch is
// bit-identical.
__device__ __forceinline__ float dpp_add(float v, int moved) { return v + __int_as_float(moved); }
__device__ __forceinline__ float wave_sum_lane63(float v) {
    v = dpp_add(v, __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    v = dpp_add(v, __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    v = dpp_add(v, __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    v = dpp_add(v, __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row_mirror
    v = dpp_add(v, __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));  // row_bcast:15
    v = dpp_add(v, __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));  // row_bcast:31
    return v;
}

__device__ __forceinline__ float dot16_s8_bf16(const v4i w, const v4i xlo, const v4i xhi, float acc) {
    // w: 16 int8; x: 16 bf16 as 8 dwords (xlo = k 0..7, xhi = k 8..15).
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t wq = (uint32_t)w[q];
        const uint32_t x01 = (uint32_t)(q < 2 ? xlo[q * 2] : xhi[(q - 2) * 2]);
        const uint32_t x23 = (uint32_t)(q < 2 ? xlo[q * 2 + 1] : xhi[(q - 2) * 2 + 1]);
        const float x0 = __uint_as_float(x01 << 16), x1 = __uint_as_float(x01 & 0xffff0000u);
        const float x2 = __uint_as_float(x23 << 16), x3 = __uint_as_float(x23 & 0xffff0000u);
        acc = __builtin_fmaf((float)(int8_t)(wq & 0xff), x0, acc);
        acc = __builtin_fmaf((float)(int8_t)((wq >> 8) & 0xff), x1, acc);
        acc = __builtin_fmaf((float)(int8_t)((wq >> 16) & 0xff), x2, acc);
        acc = __builtin_fmaf((float)(int8_t)(wq >> 24), x3, acc);
    }
    return acc;
}

// Fast path: K % 1024 == 0, 16-byte aligned rows; one wave per workgroup
// (finer dispatch than 4-wave groups: 11.9 vs 12.4 us at 14336 x 4096).
// Each wave writes its two outputs with one 4-byte store.
// CHUNKS: the K / 1024 chunk count when fixed at compile time (K = 4096),
// 0 for any.  EVEN: N % ROWS == 0 and d 4-byte aligned, so no wave clamps a
// row and each stores its two outputs with one unconditional 4-byte store
// (0.1 us less at 14336 x 4096 than the per-wave test).
template <int ROWS, int B, int CHUNKS = 0, bool EVEN = false>
__global__ __launch_bounds__(64) void gemv_s8w_m1_kernel(
    int N, int K, const uint16_t *__restrict__ x, const int8_t *__restrict__ w, int64_t ldw,
    const float *__restrict__ scale, uint16_t *__restrict__ d) {
    const int lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * ROWS;
    if (!EVEN && row0 >= N) return;
    // Rows past N (the last wave of an odd N) re-read row N - 1; wave-uniform.
    const bool whole = EVEN || row0 + ROWS <= N;
    // The row scales are requested up front: loaded after the reduction,
    // their latency would add to every wave's tail.
    float sc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) sc[r] = scale[whole ? row0 + r : min(row0 + r, N - 1)];
    const int chunks = CHUNKS ? CHUNKS : K >> 10;
    const int8_t *wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) wr[r] = w + (int64_t)(whole ? row0 + r : min(row0 + r, N - 1)) * ldw + lane * 16;
    const v4i *xv = reinterpret_cast<const v4i *>(x) + lane * 2;
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
    // Batches of B K-chunks (B divides the chunk count): every load of a
    // batch is issued before its first dot product, so a wave keeps B KiB of
    // each row in flight (one batch of 4 covers K = 4096).
    for (int c0 = 0; c0 < chunks; c0 += B) {
        v4i wv[B][ROWS], xlo[B], xhi[B];
        // The batch's x values (L2 hits) are requested before its weights:
        // loads complete in issue order, so x issued last would hold back
        // the first dot product until every weight load had landed
        // (11.27 -> 11.11 us at 14336 x 4096).
#pragma unroll
        for (int u = 0; u < B; ++u) {
            xlo[u] = xv[(c0 + u) * 128];
            xhi[u] = xv[(c0 + u) * 128 + 1];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < B; ++u)
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
                wv[u][r] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(wr[r] + (int64_t)(c0 + u) * 1024));
        // Keep the weight loads ahead of the dot products: the scheduler would
        // otherwise interleave them one load at a time.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < B; ++u)
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = dot16_s8_bf16(wv[u][r], xlo[u], xhi[u], acc[r]);
    }
    uint16_t o[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) o[r] = f32_to_bf16_rne(wave_sum_lane63(acc[r]) * sc[r]);
    if (lane == 63) {
        if (ROWS == 2 && (EVEN || (row0 + 1 < N && (reinterpret_cast<uintptr_t>(d + row0) & 3u) == 0))) {
            *reinterpret_cast<uint32_t *>(d + row0) = (uint32_t)o[0] | ((uint32_t)o[ROWS - 1] << 16);
        } else {
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
                if (row0 + r < N) d[row0 + r] = o[r];
        }
    }
}

// General path: any K, any alignment; lane l takes k = l, l+64, ... (bytes).
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_s8w_m1_generic_kernel(
    int N, int K, const uint16_t *__restrict__ x, const int8_t *__restrict__ w, int64_t ldw,
    const float *__restrict__ scale, uint16_t *__restrict__ d) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
    if (row >= N) return;
    const int8_t *wr = w + (int64_t)row * ldw;
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) acc = __builtin_fmaf((float)wr[k], bf16_to_f32(x[k]), acc);
    const float s = wave_sum(acc);
    if (lane == 0) d[row] = f32_to_bf16_rne(s * scale[row]);
}

constexpr int kGemvRows = 2;

int32_t gemv_s8w_check(int32_t n, int32_t k, int64_t ldw) {
    if (n < 0 || k < 0) return kInvalid;
    if (ldw < (k > 0 ? k : 1)) return kInvalid;
    return kOk;
}

// ---------------------------------------------------------------------------
// float gemv_dense_m1 (reference ABI)
// ---------------------------------------------------------------------------
constexpr int kDenseCols = 64;
constexpr int kDenseSlices = 16;

struct F16Tag { typedef uint16_t S; };
struct Bf16Tag { typedef uint16_t S; };

template <typename Tag> struct Codec;
template <> struct Codec<float> {
    typedef float S;
    __device__ static float ld(S v) { return v; }
    __device__ static S st(float v) { return v; }
};
template <> struct Codec<F16Tag> {
    typedef uint16_t S;
    __device__ static float ld(S v) { return f16_to_f32(v); }
    __device__ static S st(float v) { return f32_to_f16_rne(v); }
};
template <> struct Codec<Bf16Tag> {
    typedef uint16_t S;
    __device__ static float ld(S v) { return bf16_to_f32(v); }
    __device__ static S st(float v) { return f32_to_bf16_rne(v); }
};

template <typename Tag>
__global__ __launch_bounds__(kDenseCols * kDenseSlices) void gemv_dense_m1_kernel(
    int n, int k, float alpha, float beta, const typename Codec<Tag>::S *__restrict__ a,
    int64_t stride_a, const typename Codec<Tag>::S *__restrict__ b, int64_t ldb, int64_t stride_b,
    typename Codec<Tag>::S *__restrict__ d, int64_t stride_d) {
    typedef Codec<Tag> C;
    __shared__ float part[kDenseSlices][kDenseCols];
    const int slot = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int slice = threadIdx.x >> 6;
    const int j = blockIdx.x * kDenseCols + lane;
    const typename C::S *arow = a + (int64_t)slot * stride_a;
    const typename C::S *bmat = b + (int64_t)slot * stride_b;
    const int per = (k + kDenseSlices - 1) / kDenseSlices;
    const int k0 = slice * per;
    const int k1 = min(k, k0 + per);
    float acc = 0.0f;
    if (j < n) {
        for (int kk = k0; kk < k1; ++kk)
            acc = __builtin_fmaf(C::ld(arow[kk]), C::ld(bmat[(int64_t)kk * ldb + j]), acc);
    }
    part[slice][lane] = acc;
    __syncthreads();
    if (slice == 0 && j < n) {
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < kDenseSlices; ++q) s += part[q][lane];
        typename C::S *drow = d + (int64_t)slot * stride_d;
        float out = alpha * s;
        if (beta != 0.0f) out += beta * C::ld(drow[j]);
        drow[j] = C::st(out);
    }
}

// Vector path: a workgroup (16 waves) owns one column segment of 16 columns
// (64 bytes of f32, 32 bytes of f16/bf16); a lane loads 16 bytes of a B row,
// LPR = 4 (f32) / 2 (16-bit) lanes cover the segment, so one wave
// instruction reads 64 / LPR rows.  Wave w takes the K slice
// [w*per, (w+1)*per), its lanes the rows k0 + r, k0 + r + 64/LPR, ...
// (r = lane / LPR).  Partial sums are combined in a fixed order -- a
// butterfly over the row lanes, then the 16 waves in LDS -- so results are
// bit-identical from launch to launch and independent of the grid, as the
// reference's serial kernel's are.  Workgroups sharing a 128-byte line of B
// are placed on one XCD (consecutive segments per XCD).
template <typename S>
constexpr int vec_seg_bytes() { return sizeof(S) == 4 ? 64 : 32; }

template <typename Tag>
__global__ __launch_bounds__(1024) void gemv_dense_m1_vec_kernel(
    int n, int k, float alpha, float beta, const typename Codec<Tag>::S *__restrict__ a,
    int64_t stride_a, const typename Codec<Tag>::S *__restrict__ b, int64_t ldb, int64_t stride_b,
    typename Codec<Tag>::S *__restrict__ d, int64_t stride_d) {
    typedef Codec<Tag> C;
    typedef typename C::S S;
    constexpr int EPL = 16 / (int)sizeof(S);     // elements per 16-byte load
    constexpr int LPR = vec_seg_bytes<S>() / 16; // lanes per B row
    constexpr int RPI = 64 / LPR;                // rows per wave instruction
    constexpr int COLS = LPR * EPL;              // columns per workgroup
    constexpr int WAVES = 16;
    __shared__ float part[WAVES][COLS];
    const int slot = blockIdx.y;
    const int nb = gridDim.x;
    const int bx = blockIdx.x;
    const int cb = nb % 8 == 0 ? (bx % 8) * (nb / 8) + bx / 8 : bx;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane % LPR, r = lane / LPR;
    const int col = cb * COLS + q * EPL;
    const S *arow = a + (int64_t)slot * stride_a;
    const S *bmat = b + (int64_t)slot * stride_b + col;
    const int per = (k + WAVES - 1) / WAVES;
    const int k0 = wave * per;
    const int k1 = min(k, k0 + per);
    float acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.0f;
#pragma unroll 4
    for (int kk = k0 + r; kk < k1; kk += RPI) {
        const v4i w = *reinterpret_cast<const v4i *>(bmat + (int64_t)kk * ldb);
        const float av = C::ld(arow[kk]);
        if constexpr (EPL == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(av, __int_as_float(w[e]), acc[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t u = (uint32_t)w[e];
                acc[2 * e] = __builtin_fmaf(av, C::ld((S)(u & 0xffffu)), acc[2 * e]);
                acc[2 * e + 1] = __builtin_fmaf(av, C::ld((S)(u >> 16)), acc[2 * e + 1]);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) acc[e] += __shfl_xor(acc[e], off, 64);
    }
    if (r == 0) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) part[wave][q * EPL + e] = acc[e];
    }
    __syncthreads();
    if (threadIdx.x < COLS) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) sum += part[w][threadIdx.x];
        const int j = cb * COLS + threadIdx.x;
        S *drow = d + (int64_t)slot * stride_d;
        float out = alpha * sum;
        if (beta != 0.0f) out += beta * C::ld(drow[j]);
        drow[j] = C::st(out);
    }
}

// Split-K path (optional caller workspace, large problems): B read in long
// contiguous row spans instead of 32- / 64-byte column segments.  The column-
// segment pattern of the kernel above is bound by its access pattern -- a
// read-only probe of it moves the 32 MiB of a bf16 K = N = 4096 B in 16 us,
// the same bytes read contiguously take 6 us.
//   pass 1: workgroup (slice s, column group g): 256 threads x 16 bytes of
//           columns over the split_rows<Tag>() rows of slice s (16 for 16-bit
//           elements, 8 for f32); partial[s][col] =
//           sum over the slice's k (ascending) of a[k] * B[k, col]
//   pass 2: total = sum over s of partial[s][col] (16 ascending runs of
//           slices, added in run order); D = alpha * total (+ beta * D)
// Both orders are fixed, so results are bit-identical from launch to launch
// (they differ from the no-workspace kernel's order, within the same
// tolerance against the f64 reference).
// Rows per slice: more, shorter slices put more workgroups and more loads in
// flight at once; the partials grow in proportion.  K = N = 4096 with B
// rotated through HBM, one box, with workspace: bf16 8 / 12 / 16 / 24 / 32
// rows 13.6 / 14.8 / 11.0 / 17.0 / 12.1 us, f32 17.9 / 19.9 / 18.7 / 22.0 /
// 19.2 us (slice counts that are not powers of two leave ragged grids).
template <typename Tag>
constexpr int split_rows() { return sizeof(typename Codec<Tag>::S) == 4 ? 8 : 16; }
constexpr int kSplitThreads = 256;

template <typename Tag>
__global__ __launch_bounds__(kSplitThreads) void gemv_dense_split_partial_kernel(
    int n, int k, const typename Codec<Tag>::S *__restrict__ a, int64_t stride_a,
    const typename Codec<Tag>::S *__restrict__ b, int64_t ldb, int64_t stride_b, float *__restrict__ part) {
    typedef Codec<Tag> C;
    typedef typename C::S S;
    constexpr int EPL = 16 / (int)sizeof(S);
    constexpr int kSplitRows = split_rows<Tag>();
    const int slices = (k + kSplitRows - 1) / kSplitRows;
    const int s = blockIdx.x, slot = blockIdx.z;
    const int col = (blockIdx.y * kSplitThreads + threadIdx.x) * EPL;
    if (col >= n) return;
    const S *arow = a + (int64_t)slot * stride_a;
    const S *bcol = b + (int64_t)slot * stride_b + col;
    const int k0 = s * kSplitRows, k1 = min(k, k0 + kSplitRows);
    float acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.0f;
    auto fma_row = [&](const v4i &w, float av) {
        if constexpr (EPL == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(av, __int_as_float(w[e]), acc[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t u = (uint32_t)w[e];
                acc[2 * e] = __builtin_fmaf(av, C::ld((S)(u & 0xffffu)), acc[2 * e]);
                acc[2 * e + 1] = __builtin_fmaf(av, C::ld((S)(u >> 16)), acc[2 * e + 1]);
            }
        }
    };
    if (k1 - k0 == kSplitRows) {
        // whole slice (uniform branch): every row load issued before the first FMA
        v4i w[kSplitRows];
        float av[kSplitRows];
#pragma unroll
        for (int r = 0; r < kSplitRows; ++r)
            w[r] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(bcol + (int64_t)(k0 + r) * ldb));
#pragma unroll
        for (int r = 0; r < kSplitRows; ++r) av[r] = C::ld(arow[k0 + r]);
#pragma unroll
        for (int r = 0; r < kSplitRows; ++r) fma_row(w[r], av[r]);
    } else {
        for (int kk = k0; kk < k1; ++kk)
            fma_row(__builtin_nontemporal_load(reinterpret_cast<const v4i *>(bcol + (int64_t)kk * ldb)),
                    C::ld(arow[kk]));
    }
    float *dst = part + ((int64_t)slot * slices + s) * n + col;
#pragma unroll
    for (int e = 0; e < EPL; e += 4)
        *reinterpret_cast<v4f *>(dst + e) = v4f{acc[e], acc[e + 1], acc[e + 2], acc[e + 3]};
}

// Pass 2: workgroup of 16 waves per 64 columns; wave w sums the slices
// [w*per, (w+1)*per) of its lane's column in ascending order, then the 16
// wave sums are added in wave order.
template <typename Tag>
__global__ __launch_bounds__(1024) void gemv_dense_split_reduce_kernel(
    int n, int k, float alpha, float beta, const float *__restrict__ part, typename Codec<Tag>::S *__restrict__ d,
    int64_t stride_d) {
    typedef Codec<Tag> C;
    __shared__ float ws[16][64];
    constexpr int kSplitRows = split_rows<Tag>();
    const int slices = (k + kSplitRows - 1) / kSplitRows;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane, slot = blockIdx.y;
    const int per = (slices + 15) / 16;
    const int q0 = wave * per, q1 = min(slices, q0 + per);
    float s = 0.0f;
    if (j < n) {
        const float *p = part + (int64_t)slot * slices * n + j;
        int q = q0;
        for (; q + 16 <= q1; q += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = p[(int64_t)(q + u) * n];
#pragma unroll
            for (int u = 0; u < 16; ++u) s += v[u];
        }
        for (; q < q1; ++q) s += p[(int64_t)q * n];
    }
    ws[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && j < n) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; ++w) t += ws[w][lane];
        typename C::S *drow = d + (int64_t)slot * stride_d;
        float out = alpha * t;
        if (beta != 0.0f) out += beta * C::ld(drow[j]);
        drow[j] = C::st(out);
    }
}

// Workspace of the split-K path (0: the shape does not take it).  Taken for
// K >= 256 and N * K >= 2^20 elements with N a multiple of the 16-byte
// element count (and grid y / z extents within 65535); the run also needs
// 16-byte aligned B rows.
template <typename Tag>
size_t dense_split_workspace(int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout) {
    typedef typename Codec<Tag>::S S;
    constexpr int EPL = 16 / (int)sizeof(S);
    if (m != 1 || layout != 0 || n <= 0 || k < 256 || batch <= 0 || batch > 65535 || n % EPL != 0 ||
        (int64_t)n * k < (1ll << 20) || (n / EPL + kSplitThreads - 1) / kSplitThreads > 65535)
        return 0;
    const int64_t slices = (k + split_rows<Tag>() - 1) / split_rows<Tag>();
    return (size_t)batch * (size_t)slices * (size_t)n * sizeof(float);
}

// gemv_dense.cu:101-122 gemv_validate, restated.
int32_t gemv_validate(int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout, int64_t lda,
                      int64_t ldb, int64_t ldd, int64_t stride_d) {
    if (m < 0 || n < 0 || k < 0 || batch < 0) return kInvalid;
    if (m > 1) return kInvalid;
    if (layout != 0) return kInvalid;
    const int64_t min_lda = k > 0 ? k : 1;
    const int64_t min_ld_n = n > 0 ? n : 1;
    if (lda < min_lda || ldb < min_ld_n || ldd < min_ld_n) return kInvalid;
    if (batch > 1 && stride_d == 0) return kInvalid;
    return kOk;
}

template <typename Tag>
int32_t launch_dense(int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout, float alpha,
                     float beta, const void *a, int64_t lda, int64_t stride_a, const void *b,
                     int64_t ldb, int64_t stride_b, void *d, int64_t ldd, int64_t stride_d,
                     void *workspace, size_t workspace_bytes, hipStream_t stream) {
    const int32_t st = gemv_validate(m, n, k, batch, layout, lda, ldb, ldd, stride_d);
    if (st != kOk) return st;
    if (m == 0 || n == 0 || batch == 0) return kOk;
    if (!a || !b || !d) return kInvalid;
    typedef typename Codec<Tag>::S S;
    // Vector path: whole column segments and 16-byte aligned B rows (base,
    // row pitch and batch stride).
    constexpr int VCOLS = vec_seg_bytes<S>() / (int)sizeof(S);
    const bool vec = n % VCOLS == 0 && ((int64_t)ldb * (int64_t)sizeof(S)) % 16 == 0 &&
                     ((int64_t)stride_b * (int64_t)sizeof(S)) % 16 == 0 &&
                     (reinterpret_cast<uintptr_t>(b) & 15u) == 0;
    const size_t split_ws = dense_split_workspace<Tag>(m, n, k, batch, layout);
    if (split_ws != 0 && workspace != nullptr && workspace_bytes >= split_ws &&
        (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0 &&
        ((int64_t)ldb * (int64_t)sizeof(S)) % 16 == 0 && ((int64_t)stride_b * (int64_t)sizeof(S)) % 16 == 0 &&
        (reinterpret_cast<uintptr_t>(b) & 15u) == 0) {
        constexpr int EPL = 16 / (int)sizeof(S);
        const int slices = (k + split_rows<Tag>() - 1) / split_rows<Tag>();
        const int groups = (n / EPL + kSplitThreads - 1) / kSplitThreads;
        hipLaunchKernelGGL((gemv_dense_split_partial_kernel<Tag>), dim3(slices, groups, batch), dim3(kSplitThreads),
                           0, stream, n, k, (const S *)a, stride_a, (const S *)b, ldb, stride_b, (float *)workspace);
        hipLaunchKernelGGL((gemv_dense_split_reduce_kernel<Tag>), dim3((n + 63) / 64, batch), dim3(1024), 0, stream,
                           n, k, alpha, beta, (const float *)workspace, (S *)d, stride_d);
        return launch_status();
    }
    if (vec) {
        hipLaunchKernelGGL((gemv_dense_m1_vec_kernel<Tag>), dim3(n / VCOLS, batch), dim3(1024), 0, stream,
                           n, k, alpha, beta, (const S *)a, stride_a, (const S *)b, ldb, stride_b,
                           (S *)d, stride_d);
        return launch_status();
    }
    dim3 grid((n + kDenseCols - 1) / kDenseCols, batch);
    hipLaunchKernelGGL((gemv_dense_m1_kernel<Tag>), grid, dim3(kDenseCols * kDenseSlices), 0, stream,
                       n, k, alpha, beta, (const S *)a, stride_a, (const S *)b, ldb, stride_b,
                       (S *)d, stride_d);
    return launch_status();
}

}  // namespace
}  // namespace bk

using namespace bk;

extern "C" {

// ---- int8 weight-only m=1 GEMV (new SKU) ------------------------------------
int32_t baracuda_kernels_gemv_s8w_m1_bf16_gfx950_can_implement(int32_t n, int32_t k, int64_t ldw) {
    return gemv_s8w_check(n, k, ldw);
}

size_t baracuda_kernels_gemv_s8w_m1_bf16_gfx950_workspace_size(int32_t n, int32_t k) {
    (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemv_s8w_m1_bf16_gfx950_run(int32_t n, int32_t k, const void *x,
                                                     const void *w, int64_t ldw, const void *scale,
                                                     void *d, void *workspace,
                                                     size_t workspace_bytes, void *stream_ptr) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = gemv_s8w_check(n, k, ldw);
    if (st != kOk) return st;
    if (n == 0) return kOk;
    if (!x || !w || !scale || !d) return kInvalid;
    hipStream_t stream = (hipStream_t)stream_ptr;
    const bool fast = k > 0 && k % 1024 == 0 && ldw % 16 == 0 &&
                      (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    if (fast) {
        const int waves = (n + kGemvRows - 1) / kGemvRows;
        const int chunks = k / 1024;
        const bool even = n % kGemvRows == 0 && (reinterpret_cast<uintptr_t>(d) & 3u) == 0;
        if (chunks == 4 && even)
            hipLaunchKernelGGL((gemv_s8w_m1_kernel<kGemvRows, 4, 4, true>), dim3(waves), dim3(64), 0, stream, n, k,
                               (const uint16_t *)x, (const int8_t *)w, ldw, (const float *)scale, (uint16_t *)d);
        else if (chunks == 4)
            hipLaunchKernelGGL((gemv_s8w_m1_kernel<kGemvRows, 4, 4>), dim3(waves), dim3(64), 0, stream, n, k,
                               (const uint16_t *)x, (const int8_t *)w, ldw, (const float *)scale, (uint16_t *)d);
        else if (chunks % 4 == 0)
            hipLaunchKernelGGL((gemv_s8w_m1_kernel<kGemvRows, 4>), dim3(waves), dim3(64), 0, stream, n, k,
                               (const uint16_t *)x, (const int8_t *)w, ldw, (const float *)scale, (uint16_t *)d);
        else if (chunks % 2 == 0)
            hipLaunchKernelGGL((gemv_s8w_m1_kernel<kGemvRows, 2>), dim3(waves), dim3(64), 0, stream, n, k,
                               (const uint16_t *)x, (const int8_t *)w, ldw, (const float *)scale, (uint16_t *)d);
        else
            hipLaunchKernelGGL((gemv_s8w_m1_kernel<kGemvRows, 1>), dim3(waves), dim3(64), 0, stream, n, k,
                               (const uint16_t *)x, (const int8_t *)w, ldw, (const float *)scale, (uint16_t *)d);
    } else {
        hipLaunchKernelGGL(gemv_s8w_m1_generic_kernel, dim3((n + kGemvWaves - 1) / kGemvWaves),
                           dim3(64 * kGemvWaves), 0, stream, n, k, (const uint16_t *)x,
                           (const int8_t *)w, ldw, (const float *)scale, (uint16_t *)d);
    }
    return launch_status();
}

// ---- gemv_dense_m1_{f32,f16,bf16} (gemv_dense.cu:235-342 ABI) -----------------
#define BK_GEMV_DENSE(TAG, TY)                                                                    \
    int32_t baracuda_kernels_gemv_dense_m1_##TAG##_run(                                           \
        int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout, float alpha, float beta,  \
        const void *a, int64_t lda, int64_t stride_a, const void *b, int64_t ldb,                 \
        int64_t stride_b, void *d, int64_t ldd, int64_t stride_d, void *workspace,                \
        size_t workspace_bytes, void *stream) {                                                   \
        return launch_dense<TY>(m, n, k, batch, layout, alpha, beta, a, lda, stride_a, b, ldb,    \
                                stride_b, d, ldd, stride_d, workspace, workspace_bytes,           \
                                (hipStream_t)stream);                                             \
    }                                                                                             \
    int32_t baracuda_kernels_gemv_dense_m1_##TAG##_can_implement(                                 \
        int32_t m, int32_t n, int32_t k, int32_t batch, int32_t layout, int64_t lda, int64_t ldb, \
        int64_t ldd, int64_t stride_a, int64_t stride_b, int64_t stride_d) {                      \
        (void)stride_a; (void)stride_b;                                                           \
        return gemv_validate(m, n, k, batch, layout, lda, ldb, ldd, stride_d);                    \
    }                                                                                             \
    size_t baracuda_kernels_gemv_dense_m1_##TAG##_workspace_size(int32_t m, int32_t n, int32_t k, \
                                                                 int32_t batch, int32_t layout) { \
        return dense_split_workspace<TY>(m, n, k, batch, layout);                                 \
    }

BK_GEMV_DENSE(f32, float)
BK_GEMV_DENSE(f16, F16Tag)
BK_GEMV_DENSE(bf16, Bf16Tag)

#undef BK_GEMV_DENSE

}  // extern "C"
