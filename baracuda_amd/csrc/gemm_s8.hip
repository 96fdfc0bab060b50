// gemm_s8.hip -- int8 RCR GEMM SKUs for gfx950 (v_mfma_i32_16x16x64_i8).
//
// Replaces the CUTLASS int8 RCR GEMM
// (crates/baracuda-cutlass-kernels-sys/kernels/gemm_s8_rcr_sm80.cu:41-198)
// and the naive W8A8 quantized-linear kernel
// (crates/baracuda-kernels-sys/kernels/include/baracuda_quantize_compose.cuh:246-372)
// with one MFMA mainloop and four epilogues:
//   _i32      D = acc (int32)                                  new SKU
//   (plain)   D = sat_s8(rne(alpha*acc + beta*C))              gemm_s8_rcr_sm80 semantics
//   w8a8 bf16 D = bf16_rne((sa[m]*sw[n]) * (float)acc)          new SKU
//   w8a8 f32  D = (sa[m]*sw[n]) * (float)acc                    quantized_linear_w8a8_f32
//
// The accumulator wraps modulo 2^32 where the reference's mma.sync
// saturates; the two agree whenever |acc| < 2^31, which holds for int8
// operands in [-127,127] whenever K < 133143.
#include "gemm_mfma.hpp"
#include "gemm_mfma2.hpp"

namespace bk {
namespace {

using namespace mfma;

enum Epi : int { EPI_I32 = 0, EPI_S8 = 1, EPI_W8A8_BF16 = 2, EPI_W8A8_F32 = 3 };

struct S8Args {
    int M, N, K;
    const int8_t *a; int64_t lda;
    const int8_t *b; int64_t ldb;
    const int8_t *c; int64_t ldc;
    void *d; int64_t ldd;
    float alpha, beta;
    const float *sa; const float *sw;
};

// Epilogue on one group of 4 consecutive output columns of row m.
template <int EPI, bool VecOut>
struct S8Epilogue {
    const S8Args &p;
    __device__ __forceinline__ void operator()(int m, int n0, const v4i &v) const {
        if (m >= p.M || n0 >= p.N) return;
        // VecOut implies N % 4 == 0, so a group is then always complete.
        const int count = VecOut ? 4 : (p.N - n0 < 4 ? p.N - n0 : 4);
        const bool vec = VecOut;
        if constexpr (EPI == EPI_I32) {
            int32_t *d = static_cast<int32_t *>(p.d) + (int64_t)m * p.ldd + n0;
            if (vec) *reinterpret_cast<v4i *>(d) = v;
            else for (int r = 0; r < count; ++r) d[r] = v[r];
        } else if constexpr (EPI == EPI_S8) {
            // gemm_s8_rcr_sm80 epilogue: z = alpha*acc + beta*C, RNE, clamp.
            int8_t *d = static_cast<int8_t *>(p.d) + (int64_t)m * p.ldd + n0;
            int8_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float z = p.alpha * (float)v[r];
                if (p.beta != 0.0f && p.c != nullptr && r < count)
                    z += p.beta * (float)p.c[(int64_t)m * p.ldc + n0 + r];
                o[r] = sat_cast_s8(z);
            }
            if (vec) {
                uint32_t w = (uint32_t)(uint8_t)o[0] | ((uint32_t)(uint8_t)o[1] << 8) |
                             ((uint32_t)(uint8_t)o[2] << 16) | ((uint32_t)(uint8_t)o[3] << 24);
                *reinterpret_cast<uint32_t *>(d) = w;
            } else {
                for (int r = 0; r < count; ++r) d[r] = o[r];
            }
        } else {
            // W8A8 dequant: y = (sa[m] * sw[n]) * (float)acc, products in f32.
            const float sam = p.sa[m];
            float y[4];
            if (vec) {
                const v4f sw = *reinterpret_cast<const v4f *>(p.sw + n0);
#pragma unroll
                for (int r = 0; r < 4; ++r) y[r] = (sam * sw[r]) * (float)v[r];
            } else {
                for (int r = 0; r < 4; ++r) y[r] = r < count ? (sam * p.sw[n0 + r]) * (float)v[r] : 0.0f;
            }
            if constexpr (EPI == EPI_W8A8_BF16)
                store4_bf16(static_cast<uint16_t *>(p.d) + (int64_t)m * p.ldd + n0, y, vec, count);
            else
                store4_f32(static_cast<float *>(p.d) + (int64_t)m * p.ldd + n0, y, vec, count);
        }
    }
};

// General path: register-staged mainloop (K tail / unaligned operands).
template <int EPI, bool VecOut>
__global__ __launch_bounds__(NT, 1) void gemm_s8_rcr_kernel(S8Args p) {
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
    v4i acc[TM][TN];
    mainloop<Elem::S8, true>(lds, as, bs, p.K, acc);
    const S8Epilogue<EPI, VecOut> epi{p};
    for_each_fragment(acc, [&](int ml, int nl, const v4i &v) { epi(m_base + ml, n_base + nl, v); });
}

// Fast path: M, N multiples of 256, K % 128 == 0, 16-byte aligned rows ->
// LDS-DMA mainloop, 8 waves (2 x 4) of 128 x 64, v_mfma_i32_16x16x64_i8.
typedef mfma2::Cfg<2, 4, 0> DmaCfg;

template <int EPI, bool VecOut>
__global__ __launch_bounds__(DmaCfg::NT, 1) void gemm_s8_rcr_dma_kernel(S8Args p) {
    namespace M2 = mfma2;
    typedef M2::PolicyI8<DmaCfg> P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * M2::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * M2::OPER];
    const int tiles_m = p.M / M2::BM, tiles_n = p.N / M2::BN;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m_base = tm * M2::BM, n_base = tn * M2::BN;
    M2::DmaRows<false, false> d;
    d.a = M2::make_dma_interior<DmaCfg>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
    d.b = M2::make_dma_interior<DmaCfg>(p.b, (uint32_t)(p.N * p.ldb), (int)p.ldb, n_base * (int)p.ldb);
    M2::AccTile<P> acc;
    M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    if constexpr (EPI == EPI_W8A8_BF16 && VecOut) {
        // Whole tiles: scales fetched once per lane, output staged in LDS
        // (free after the mainloop's last barrier) and written as full rows.
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wrow = m_base + (wave / DmaCfg::WAVES_N) * DmaCfg::WM;
        const int wcol = n_base + (wave % DmaCfg::WAVES_N) * DmaCfg::WN;
        float sam[P::TI], none[P::TI];
        v4f swv[P::TJ];
#pragma unroll
        for (int i = 0; i < P::TI; ++i) sam[i] = p.sa[wrow + i * 16 + (lane & 15)];
#pragma unroll
        for (int j = 0; j < P::TJ; ++j)
            swv[j] = *reinterpret_cast<const v4f *>(p.sw + wcol + j * 16 + (lane >> 4) * 4);
        int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (DmaCfg::WM * DmaCfg::WN * 2);
        M2::store_w8a8_bf16_staged<P, false>(acc, scratch, sam, none, swv, [&](int r) {
            return static_cast<uint16_t *>(p.d) + (int64_t)(wrow + r) * p.ldd + wcol;
        });
    } else {
        const S8Epilogue<EPI, VecOut> epi{p};
        M2::for_each_quad<P>(acc, [&](int ml, int nl, const v4i &v) { epi(m_base + ml, n_base + nl, v); });
    }
}

template <int EPI, bool VecOut>
void launch_kernel(const S8Args &p, bool fast_k, hipStream_t stream) {
    if (fast_k) {
        const int tiles = ((p.M + mfma2::BM - 1) / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
        hipLaunchKernelGGL((gemm_s8_rcr_dma_kernel<EPI, VecOut>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, p);
    } else {
        const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
        hipLaunchKernelGGL((gemm_s8_rcr_kernel<EPI, VecOut>), dim3(tiles), dim3(NT), 0, stream, p);
    }
}

template <int EPI>
int32_t launch(const S8Args &p, hipStream_t stream) {
    const int out_elem = (EPI == EPI_I32 || EPI == EPI_W8A8_F32) ? 4 : (EPI == EPI_S8 ? 1 : 2);
    // The DMA path needs whole 256x256 tiles, whole K stages and 16-byte rows.
    const bool fast_k = p.K > 0 && p.K % BK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 &&
                        aligned16(p.a) && aligned16(p.b) &&
                        (int64_t)p.M * p.lda < (1ll << 31) && (int64_t)p.N * p.ldb < (1ll << 31) &&
                        p.M % mfma2::BM == 0 && p.N % mfma2::BN == 0;
    // 4-wide vector stores need every 4-column group of D (and sw) aligned;
    // the LDS-staged W8A8 bf16 store writes 16-byte units (8 columns).
    bool vec = ((p.ldd * out_elem) % (4 * out_elem)) == 0 &&
               (reinterpret_cast<uintptr_t>(p.d) % (4 * out_elem)) == 0 &&
               (p.sw == nullptr || aligned16(p.sw)) && (p.N % 4 == 0);
    if (EPI == EPI_W8A8_BF16) vec = vec && p.ldd % 8 == 0 && aligned16(p.d);
    if (vec) launch_kernel<EPI, true>(p, fast_k, stream);
    else launch_kernel<EPI, false>(p, fast_k, stream);
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

// ---- int8 RCR, int32 output (new SKU) -------------------------------------
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return check_rcr(m, n, k, lda, ldb, ldd);
}

size_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_s8_rcr_gfx950_i32_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    void *d, int64_t ldd, void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd,
             1.0f, 0.0f, nullptr, nullptr};
    return launch<EPI_I32>(p, (hipStream_t)stream);
}

// ---- int8 RCR, int8 output: D = sat_s8(alpha*acc + beta*C) ------------------
// Same ABI as baracuda_kernels_gemm_s8_rcr_sm80_* (gemm_s8_rcr_sm80.cu:169-198).
int32_t baracuda_kernels_gemm_s8_rcr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (c != nullptr && ldc < n) return kInvalid;
    return kOk;
}

size_t baracuda_kernels_gemm_s8_rcr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_s8_rcr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = baracuda_kernels_gemm_s8_rcr_gfx950_can_implement(m, n, k, a, lda, b, ldb, c, ldc, d, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, ldd,
             alpha, beta, nullptr, nullptr};
    return launch<EPI_S8>(p, (hipStream_t)stream);
}

// ---- W8A8: D = bf16((scale_a[m] * scale_b[n]) * acc) (new SKU) -----------
int32_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *scale_a, const void *scale_b, const void *d, int64_t ldd) {
    (void)a; (void)b; (void)scale_a; (void)scale_b; (void)d;
    return check_rcr(m, n, k, lda, ldb, ldd);
}

size_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_workspace_size(int32_t m, int32_t n, int32_t k) {
    (void)m; (void)n; (void)k;
    return 0;
}

int32_t baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const float *scale_a, const float *scale_b, void *d, int64_t ldd,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    int32_t st = check_rcr(m, n, k, lda, ldb, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d || !scale_a || !scale_b) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, nullptr, 0, d, ldd,
             1.0f, 0.0f, scale_a, scale_b};
    return launch<EPI_W8A8_BF16>(p, (hipStream_t)stream);
}

// ---- quantized_linear_w8a8 f32 (baracuda_quantize_compose.cuh:340-370 ABI) --
// y[m, c] = scale_a[m] * scale_w[c] * acc, weight [C_out, K], act [M, K].
int32_t baracuda_kernels_quantized_linear_w8a8_f32_gfx950_can_implement(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, const void *output) {
    (void)weight_q; (void)act_q; (void)scale_a; (void)scale_w; (void)output;
    if (M < 0 || C_out < 0 || K < 0) return kInvalid;
    return kOk;
}

int32_t baracuda_kernels_quantized_linear_w8a8_f32_gfx950_run(
    int32_t M, int32_t C_out, int32_t K, const void *weight_q, const void *act_q,
    const void *scale_a, const void *scale_w, void *output,
    void *workspace, size_t workspace_bytes, void *stream) {
    (void)workspace; (void)workspace_bytes;
    if (M < 0 || C_out < 0 || K < 0) return kInvalid;
    if ((int64_t)M * C_out == 0) return kOk;
    if (!weight_q || !act_q || !scale_a || !scale_w || !output) return kInvalid;
    if (K == 0) {
        // Empty reduction: acc = 0 for every cell, handled by a K=0 tile pass.
        S8Args p{M, C_out, 0, (const int8_t *)act_q, 0, (const int8_t *)weight_q, 0, nullptr, 0,
                 output, C_out, 1.0f, 0.0f, (const float *)scale_a, (const float *)scale_w};
        return launch<EPI_W8A8_F32>(p, (hipStream_t)stream);
    }
    S8Args p{M, C_out, K, (const int8_t *)act_q, K, (const int8_t *)weight_q, K, nullptr, 0,
             output, C_out, 1.0f, 0.0f, (const float *)scale_a, (const float *)scale_w};
    return launch<EPI_W8A8_F32>(p, (hipStream_t)stream);
}

}  // extern "C"
