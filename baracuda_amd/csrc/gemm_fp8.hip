// gemm_fp8.hip -- FP8 E4M3 (OCP e4m3fn) RCR GEMM SKUs for gfx950, both
// operands e4m3, f32 accumulator (v_mfma_f32_32x32x64_f8f6f4 on the LDS-DMA
// path for whole 256x256 tiles, v_mfma_f32_16x16x128_f8f6f4 on the general
// path).
//
// Replaces baracuda_kernels_gemm_fp8_e4m3_rcr_sm89_*
// (crates/baracuda-kernels-sys/kernels/gemm/gemm_fp8_e4m3_rcr_sm89.cu:31-67,
//  kernel crates/baracuda-kernels-sys/kernels/include/baracuda_fp8_rcr_sm89.cuh:102-323):
//   (plain)  D = sat_e4m3(alpha*acc + beta*dequant(C))     reference semantics, e4m3 out
//   _bf16    D = bf16_rne((scale_a*scale_b) * acc)          new SKU (per-tensor scales)
//   _f32     D = alpha * acc                                 new SKU (accumulator check)
#include "gemm_mfma.hpp"
#include "gemm_mfma2.hpp"

namespace bk {
namespace {

using namespace mfma;

enum Epi : int { EPI_E4M3 = 0, EPI_BF16 = 1, EPI_F32 = 2 };

struct F8Args {
    int M, N, K;
    const int8_t *a; int64_t lda;
    const int8_t *b; int64_t ldb;
    const uint8_t *c; int64_t ldc;
    void *d; int64_t ldd;
    float alpha, beta;
};

// Epilogue on one group of 4 consecutive output columns of row m.
template <int EPI, bool VecOut>
struct F8Epilogue {
    const F8Args &p;
    __device__ __forceinline__ void operator()(int m, int n0, const v4f &v) const {
        if (m >= p.M || n0 >= p.N) return;
        const int count = VecOut ? 4 : (p.N - n0 < 4 ? p.N - n0 : 4);
        const bool vec = VecOut;
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = p.alpha * v[r];
        if constexpr (EPI == EPI_E4M3) {
            uint8_t *d = static_cast<uint8_t *>(p.d) + (int64_t)m * p.ldd + n0;
            uint8_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float z = y[r];
                if (p.beta != 0.0f && p.c != nullptr && r < count)
                    z += p.beta * e4m3_to_f32(p.c[(int64_t)m * p.ldc + n0 + r]);
                o[r] = f32_to_e4m3_satfinite(z);
            }
            if (vec) {
                *reinterpret_cast<uint32_t *>(d) = (uint32_t)o[0] | ((uint32_t)o[1] << 8) |
                                                   ((uint32_t)o[2] << 16) | ((uint32_t)o[3] << 24);
            } else {
                for (int r = 0; r < count; ++r) d[r] = o[r];
            }
        } else if constexpr (EPI == EPI_BF16) {
            store4_bf16(static_cast<uint16_t *>(p.d) + (int64_t)m * p.ldd + n0, y, vec, count);
        } else {
            store4_f32(static_cast<float *>(p.d) + (int64_t)m * p.ldd + n0, y, vec, count);
        }
    }
};

// General path: register-staged mainloop (K tail / unaligned / partial tiles).
template <int EPI, bool VecOut>
__global__ __launch_bounds__(NT, 1) void gemm_fp8_rcr_kernel(F8Args p) {
    __shared__ __attribute__((aligned(16))) int8_t lds[4 * LDS_TILE];
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m_base = tm * BM, n_base = tn * BN;
    const int tid = threadIdx.x;
    RowSet as, bs;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int r = i * LOAD_ROWS + (tid >> 3);
        const int am = min(m_base + r, p.M - 1), bn = min(n_base + r, p.N - 1);
        as.ptr[i] = p.a + (int64_t)am * p.lda;
        bs.ptr[i] = p.b + (int64_t)bn * p.ldb;
    }
    v4f acc[TM][TN];
    mainloop<Elem::E4M3, true>(lds, as, bs, p.K, acc);
    const F8Epilogue<EPI, VecOut> epi{p};
    for_each_fragment(acc, [&](int ml, int nl, const v4f &v) { epi(m_base + ml, n_base + nl, v); });
}

// Fast path: whole 256x256 tiles, K % 128 == 0, 16-byte rows -> LDS-DMA
// mainloop, 8 waves (2 x 4) of 128 x 64, v_mfma_f32_32x32x64_f8f6f4.
typedef mfma2::Cfg<2, 4, 0> DmaCfg;

template <int EPI, bool VecOut>
__global__ __launch_bounds__(DmaCfg::NT, 1) void gemm_fp8_rcr_dma_kernel(F8Args p) {
    namespace M2 = mfma2;
    typedef M2::PolicyF8<DmaCfg> P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * M2::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * M2::OPER];
    int tm, tn;
    tile_coords(blockIdx.x, p.M / M2::BM, p.N / M2::BN, tm, tn);
    const int m_base = tm * M2::BM, n_base = tn * M2::BN;
    M2::DmaRows<false, false> d;
    d.a = M2::make_dma_interior<DmaCfg>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
    d.b = M2::make_dma_interior<DmaCfg>(p.b, (uint32_t)(p.N * p.ldb), (int)p.ldb, n_base * (int)p.ldb);
    M2::AccTile<P> acc;
    M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    const F8Epilogue<EPI, VecOut> epi{p};
    M2::for_each_quad<P>(acc, [&](int ml, int nl, const v4f &v) { epi(m_base + ml, n_base + nl, v); });
}

template <int EPI, bool VecOut>
void launch_kernel(const F8Args &p, bool fast, hipStream_t stream) {
    if (fast) {
        const int tiles = (p.M / mfma2::BM) * (p.N / mfma2::BN);
        hipLaunchKernelGGL((gemm_fp8_rcr_dma_kernel<EPI, VecOut>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, p);
    } else {
        const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
        hipLaunchKernelGGL((gemm_fp8_rcr_kernel<EPI, VecOut>), dim3(tiles), dim3(NT), 0, stream, p);
    }
}

template <int EPI>
int32_t launch(const F8Args &p, hipStream_t stream) {
    const int out_elem = EPI == EPI_F32 ? 4 : (EPI == EPI_BF16 ? 2 : 1);
    // The DMA path needs whole 256x256 tiles, whole K stages and 16-byte rows.
    const bool fast = p.K % BK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.a) &&
                      aligned16(p.b) && p.M % mfma2::BM == 0 && p.N % mfma2::BN == 0 &&
                      (int64_t)p.M * p.lda < (1ll << 31) && (int64_t)p.N * p.ldb < (1ll << 31);
    const bool vec = p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % (4 * out_elem)) == 0 &&
                     p.N % 4 == 0;
    if (vec) launch_kernel<EPI, true>(p, fast, stream);
    else launch_kernel<EPI, false>(p, fast, stream);
    return launch_status();
}

int32_t check_rcr(int32_t m, int32_t n, int32_t k, int64_t lda, int64_t ldb, int64_t ldd) {
    if (m <= 0 || n <= 0 || k <= 0) return kInvalid;
    if (lda < k || ldb < k || ldd < n) return kInvalid;
    return kOk;
}

}  // namespace
}  // namespace bk

using namespace bk;

extern "C" {

// ---- e4m3 out: D = sat_e4m3(alpha*acc + beta*dequant(C)) (sm89 ABI) --------
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, const void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (c != nullptr && ldc < n) return kInvalid;
    return kOk;
}

size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_can_implement(m, n, k, a, lda, b, ldb, c, ldc, d, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    F8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const uint8_t *)c, ldc, d, ldd,
             alpha, beta};
    return launch<EPI_E4M3>(p, (hipStream_t)stream);
}

// ---- bf16 out with per-tensor scales (new SKU) ------------------------------
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return check_rcr(m, n, k, lda, ldb, ldd);
}

size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    float scale_a, float scale_b, void *d, int64_t ldd,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    F8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd,
             scale_a * scale_b, 0.0f};
    return launch<EPI_BF16>(p, (hipStream_t)stream);
}

// ---- f32 out: D = alpha * acc (new SKU, exposes the accumulator) ------------
int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return check_rcr(m, n, k, lda, ldb, ldd);
}

size_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    float alpha, void *d, int64_t ldd, void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    F8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd, alpha, 0.0f};
    return launch<EPI_F32>(p, (hipStream_t)stream);
}

}  // extern "C"
