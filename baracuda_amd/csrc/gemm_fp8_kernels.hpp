// gemm_fp8_kernels.hpp -- the FP8 GEMM kernels and launchers shared by the
// FP8 SKU translation units (gemm_fp8.hip, gemm_fp8_bias.hip,
// gemm_fp8_bias_e5m2.hip).
//
// Operands e4m3 (FMT_E4M3) or e5m2 (FMT_E5M2), both of one encoding; A
// row-major [M,K]; B [N,K] (RCR) or row-major [K,N] (RRR); f32 accumulator.
// Outputs:
//   F8_OUT   D = sat_fp8(act(alpha*acc + beta*dec(C) [+ bias[n]]))   reference SKUs
//   F8_BF16  D = bf16_rne(alpha * acc)                                 new SKU
//   F8_F32   D = alpha * acc                                           new SKU
// (baracuda_fp8_rcr_sm89.cuh:102-323, baracuda_fp8_rrr_sm89.cuh:60-272).
//
// Whole 256x256 tiles with K % 128 == 0 and 16-byte rows take the LDS-DMA
// mainloop (v_mfma_f32_32x32x64_f8f6f4; RRR reads B with transposing LDS
// reads); everything else the register-staged mainloop (16x16x128).
#pragma once

#include <type_traits>

#include "gemm_mfma.hpp"
#include "gemm_mfma2.hpp"
#include "act.hpp"

namespace bk {
namespace {

using namespace mfma;

enum F8Epi : int { F8_OUT = 0, F8_BF16 = 1, F8_F32 = 2 };
enum F8Layout : int { F8_RCR = 0, F8_RRR = 1 };

struct F8Args {
    int M, N, K;
    const int8_t *a; int64_t lda;
    const int8_t *b; int64_t ldb;
    const uint8_t *c; int64_t ldc;
    void *d; int64_t ldd;
    float alpha, beta;
    const float *bias;   // [N], for ACT != ACT_NONE
};

// Epilogue on one group of 4 consecutive output columns of row m.
template <int FMT, int EPI, bool VecOut, int ACT>
struct F8Epilogue {
    const F8Args &p;
    // F8_OUT, whole group of 4 columns (N % 4 == 0): the 4 result bytes.
    // HasC: beta != 0 and C given; CVec: the 4 C bytes read as one dword
    // (ldc and C 4-byte aligned) -- both decided once per tile by the caller.
    template <bool HasC, bool CVec = false>
    __device__ __forceinline__ uint32_t pack_fp8(int m, int n0, const v4f &v) const {
        float z[4];
        uint32_t c4 = 0;
        if constexpr (HasC && CVec) c4 = *reinterpret_cast<const uint32_t *>(p.c + (int64_t)m * p.ldc + n0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            z[r] = p.alpha * v[r];
            if constexpr (HasC) {
                const uint8_t cb = CVec ? (uint8_t)(c4 >> (8 * r)) : p.c[(int64_t)m * p.ldc + n0 + r];
                z[r] += p.beta * fp8_to_f32<FMT>(cb);
            }
            if constexpr (ACT != ACT_NONE) {
                z[r] += p.bias[n0 + r];
                z[r] = activation<ACT>(z[r]);
            }
        }
        return f32x4_to_fp8x4_satfinite<FMT>(z[0], z[1], z[2], z[3]);
    }
    __device__ __forceinline__ void operator()(int m, int n0, const v4f &v) const {
        if (m >= p.M || n0 >= p.N) return;
        const int count = VecOut ? 4 : (p.N - n0 < 4 ? p.N - n0 : 4);
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = p.alpha * v[r];
        if constexpr (EPI == F8_OUT) {
            uint8_t *d = static_cast<uint8_t *>(p.d) + (int64_t)m * p.ldd + n0;
            float z[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                z[r] = y[r];
                if (p.beta != 0.0f && p.c != nullptr && r < count)
                    z[r] += p.beta * fp8_to_f32<FMT>(p.c[(int64_t)m * p.ldc + n0 + r]);
                if constexpr (ACT != ACT_NONE) {
                    if (r < count) z[r] += p.bias[n0 + r];
                    z[r] = activation<ACT>(z[r]);
                }
            }
            const uint32_t w = f32x4_to_fp8x4_satfinite<FMT>(z[0], z[1], z[2], z[3]);
            if constexpr (VecOut) {
                *reinterpret_cast<uint32_t *>(d) = w;
            } else {
                for (int r = 0; r < count; ++r) d[r] = (uint8_t)(w >> (8 * r));
            }
        } else if constexpr (EPI == F8_BF16) {
            store4_bf16(static_cast<uint16_t *>(p.d) + (int64_t)m * p.ldd + n0, y, VecOut, count);
        } else {
            store4_f32(static_cast<float *>(p.d) + (int64_t)m * p.ldd + n0, y, VecOut, count);
        }
    }
};

// General path: register-staged mainloop (K tail / unaligned / partial tiles).
template <int FMT, int LAYOUT, int EPI, int ACT>
__global__ __launch_bounds__(NT, 1) void gemm_fp8_kernel(F8Args p) {
    constexpr Elem E = FMT == FMT_E5M2 ? Elem::E5M2 : Elem::E4M3;
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
        as.ptr[i] = p.a + (int64_t)min(m_base + r, p.M - 1) * p.lda;
        bs.ptr[i] = p.b + (int64_t)min(n_base + r, p.N - 1) * p.ldb;
    }
    v4f acc[TM][TN];
    if constexpr (LAYOUT == F8_RCR) mainloop<E, true>(lds, as, bs, p.K, acc);
    else mainloop_rrr<E, true, true>(lds, as, p.b, p.ldb, p.N, n_base, p.K, acc);
    const F8Epilogue<FMT, EPI, false, ACT> epi{p};
    for_each_fragment(acc, [&](int ml, int nl, const v4f &v) { epi(m_base + ml, n_base + nl, v); });
}

typedef mfma2::Cfg<2, 4> F8DmaCfg;

template <int FMT, int LAYOUT>
struct F8DmaPolicy { typedef mfma2::PolicyF8<F8DmaCfg, FMT> type; };
template <int FMT>
struct F8DmaPolicy<FMT, F8_RRR> { typedef mfma2::PolicyF8RowB<F8DmaCfg, FMT> type; };

// Fast path: 256x256 tiles (edge tiles included), K % 128 == 0, 16-byte rows,
// N % 4 == 0, vector stores.
template <int FMT, int LAYOUT, int EPI, int ACT>
__global__ __launch_bounds__(F8DmaCfg::NT, 1) void gemm_fp8_dma_kernel(F8Args p) {
    namespace M2 = mfma2;
    typedef typename F8DmaPolicy<FMT, LAYOUT>::type P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * M2::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * M2::OPER];
    // Edge tiles (M or N not a multiple of 256): rows past M / N load as
    // zeros (past the buffer resources' byte counts; RRR B columns past N
    // read the next k-row, reaching only output columns that are not stored).
    int tm, tn;
    tile_coords(blockIdx.x, (p.M + M2::BM - 1) / M2::BM, (p.N + M2::BN - 1) / M2::BN, tm, tn);
    const int m_base = tm * M2::BM, n_base = tn * M2::BN;
    const bool full = m_base + M2::BM <= p.M && n_base + M2::BN <= p.N;
    M2::AccTile<P> acc;
    if constexpr (LAYOUT == F8_RCR) {
        M2::DmaRows<false, false> d;
        d.a = M2::make_dma_interior<F8DmaCfg>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
        d.b = M2::make_dma_interior<F8DmaCfg>(p.b, (uint32_t)(p.N * p.ldb), (int)p.ldb, n_base * (int)p.ldb);
        M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    } else {
        M2::DmaRowsRrr d;
        d.a = M2::make_dma_interior<F8DmaCfg>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
        d.b = M2::make_dma_row_b<F8DmaCfg>(p.b, (uint32_t)(p.K * p.ldb), (int)p.ldb, n_base);
        M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    }
    if constexpr (EPI == F8_BF16) {
        // bf16 rows staged per wave in LDS (free after the mainloop's last
        // barrier), written as 16-byte units: D = bf16_rne(alpha * acc).
        if (p.ldd % 8 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 8 == 0)) {
            const int wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / F8DmaCfg::WAVES_N) * F8DmaCfg::WM;
            const int wcol = n_base + (wave % F8DmaCfg::WAVES_N) * F8DmaCfg::WN;
            int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (F8DmaCfg::WM * 128);
            const float alpha = p.alpha;
            M2::store_bf16x4_staged<P>(
                acc, scratch,
                [&](int, int, const v4f &v) {
                    return v2i{(int)f32x2_to_bf16x2(alpha * v[0], alpha * v[1]),
                               (int)f32x2_to_bf16x2(alpha * v[2], alpha * v[3])};
                },
                [&](int r) {
                    return wrow + r < p.M ? static_cast<uint16_t *>(p.d) + (int64_t)(wrow + r) * p.ldd + wcol
                                          : nullptr;
                },
                min(F8DmaCfg::WN, p.N - wcol));
            return;
        }
    }
    if constexpr (EPI == F8_F32) {
        // f32 rows staged in LDS (two halves) and written as 256-byte row
        // segments: D = alpha * acc.
        if (p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 4 == 0)) {
            const int wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / F8DmaCfg::WAVES_N) * F8DmaCfg::WM;
            const int wcol = n_base + (wave % F8DmaCfg::WAVES_N) * F8DmaCfg::WN;
            int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (F8DmaCfg::WM / 2 * 256);
            const float alpha = p.alpha;
            M2::store_x32x4_staged<P>(
                acc, scratch,
                [&](int, int, const v4f &v) {
                    return v4i{__float_as_int(alpha * v[0]), __float_as_int(alpha * v[1]),
                               __float_as_int(alpha * v[2]), __float_as_int(alpha * v[3])};
                },
                [&](int r) {
                    return wrow + r < p.M ? static_cast<float *>(p.d) + (int64_t)(wrow + r) * p.ldd + wcol : nullptr;
                },
                min(F8DmaCfg::WN, p.N - wcol));
            return;
        }
    }
    const F8Epilogue<FMT, EPI, true, ACT> epi{p};
    if constexpr (EPI == F8_OUT) {
        // fp8 bytes staged per wave, written as 16-byte row segments.
        if (p.ldd % 16 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 16 == 0)) {
            const int wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / F8DmaCfg::WAVES_N) * F8DmaCfg::WM;
            const int wcol = n_base + (wave % F8DmaCfg::WAVES_N) * F8DmaCfg::WN;
            int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (F8DmaCfg::WM * F8DmaCfg::WN);
            // The C term and the M / N bounds decided once per tile, not per element.
            auto staged = [&](auto has_c, auto whole) {
                M2::store_u8x4_staged<P>(
                    acc, scratch,
                    [&](int r, int c, const v4f &v) {
                        // whole tiles with C: C rows read as dwords when aligned
                        constexpr bool kC = decltype(has_c)::value, kW = decltype(whole)::value;
                        if constexpr (kW)
                            return epi.template pack_fp8<kC, kC>(wrow + r, wcol + c, v);
                        else
                            return (wrow + r < p.M && wcol + c < p.N)
                                       ? epi.template pack_fp8<kC>(wrow + r, wcol + c, v)
                                       : 0u;
                    },
                    [&](int r) {
                        return wrow + r < p.M ? static_cast<int8_t *>(p.d) + (int64_t)(wrow + r) * p.ldd + wcol
                                              : nullptr;
                    },
                    min(F8DmaCfg::WN, p.N - wcol));
            };
            using T_ = std::true_type;
            using F_ = std::false_type;
            const bool has_c = p.beta != 0.0f && p.c != nullptr;
            const bool c_vec = p.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(p.c) & 3u) == 0;
            if (has_c) {
                if (full && c_vec) staged(T_{}, T_{});
                else staged(T_{}, F_{});
            } else {
                if (full) staged(F_{}, T_{});
                else staged(F_{}, F_{});
            }
            return;
        }
    }
    M2::for_each_quad<P>(acc, [&](int ml, int nl, const v4f &v) { epi(m_base + ml, n_base + nl, v); });
}

template <int FMT, int LAYOUT, int EPI, int ACT>
int32_t launch_fp8(const F8Args &p, hipStream_t stream) {
    const int out_elem = EPI == F8_F32 ? 4 : (EPI == F8_BF16 ? 2 : 1);
    const int64_t b_rows = LAYOUT == F8_RCR ? p.N : p.K;
    // Edge tiles load zeros past the operands, so the byte offsets of the
    // extents padded to whole tiles must stay below 2^31; the vector epilogue
    // needs whole 4-column groups (N % 4 == 0).
    const int64_t pad_m = (int64_t)((p.M + mfma2::BM - 1) / mfma2::BM) * mfma2::BM;
    const int64_t pad_b = LAYOUT == F8_RCR ? (int64_t)((p.N + mfma2::BN - 1) / mfma2::BN) * mfma2::BN * p.ldb
                                           : b_rows * p.ldb + mfma2::BN;
    const bool fast = p.K % mfma2::BK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.a) &&
                      aligned16(p.b) && p.N % 4 == 0 && pad_m * p.lda < (1ll << 31) && pad_b < (1ll << 31) &&
                      p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % (4 * out_elem)) == 0;
    if (fast) {
        const int tiles = (int)(pad_m / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
        hipLaunchKernelGGL((gemm_fp8_dma_kernel<FMT, LAYOUT, EPI, ACT>), dim3(tiles), dim3(F8DmaCfg::NT),
                           0, stream, p);
    } else {
        const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
        hipLaunchKernelGGL((gemm_fp8_kernel<FMT, LAYOUT, EPI, ACT>), dim3(tiles), dim3(NT), 0, stream, p);
    }
    return launch_status();
}

// Extent / leading-dimension checks of the reference launchers plus the
// row-length bounds the kernels index with: B rows are K bytes (RCR) or N
// bytes (RRR).
template <int LAYOUT>
int32_t check_fp8(int32_t m, int32_t n, int32_t k, int64_t lda, int64_t ldb, const void *c,
                  int64_t ldc, int64_t ldd) {
    if (m <= 0 || n <= 0 || k <= 0) return kInvalid;
    if (lda < k || ldd < n) return kInvalid;
    if (ldb < (LAYOUT == F8_RCR ? k : n)) return kInvalid;
    if (c != nullptr && ldc < n) return kInvalid;
    return kOk;
}

}  // namespace
}  // namespace bk

// Entry points of one fp8-out SKU: baracuda_kernels_gemm_fp8_<ENC>_<LAY>_gfx950[_<EPI>]_*.
#define BK_FP8_IDENTITY_SKU(ENC, LAY, FMT, LAYOUT)                                                 \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_can_implement(                        \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,    \
        const void *c, int64_t ldc, const void *d, int64_t ldd) {                                   \
        (void)a; (void)b; (void)d;                                                                  \
        return bk::check_fp8<LAYOUT>(m, n, k, lda, ldb, c, ldc, ldd);                               \
    }                                                                                               \
    size_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_workspace_size(int32_t m, int32_t n,   \
                                                                          int32_t k) {             \
        (void)m; (void)n; (void)k;                                                                  \
        return 0;                                                                                   \
    }                                                                                               \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_run(                                  \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,    \
        const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,                  \
        void *workspace, size_t workspace_bytes, void *stream) {                                    \
        (void)workspace; (void)workspace_bytes;                                                     \
        int32_t st = bk::check_fp8<LAYOUT>(m, n, k, lda, ldb, c, ldc, ldd);                         \
        if (st != bk::kOk) return st;                                                               \
        if (!a || !b || !d) return bk::kInvalid;                                                    \
        bk::F8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const uint8_t *)c,   \
                     ldc, d, ldd, alpha, beta, nullptr};                                            \
        return bk::launch_fp8<FMT, LAYOUT, bk::F8_OUT, bk::ACT_NONE>(p, (hipStream_t)stream);       \
    }

#define BK_FP8_BIAS_SKU(ENC, LAY, EPISFX, FMT, LAYOUT, ACTV)                                       \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_##EPISFX##_can_implement(              \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,    \
        const void *c, int64_t ldc, const void *d, int64_t ldd) {                                   \
        (void)a; (void)b; (void)d;                                                                  \
        return bk::check_fp8<LAYOUT>(m, n, k, lda, ldb, c, ldc, ldd);                               \
    }                                                                                               \
    int32_t baracuda_kernels_gemm_fp8_##ENC##_##LAY##_gfx950_##EPISFX##_run(                        \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,    \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha,            \
        float beta, void *workspace, size_t workspace_bytes, void *stream) {                        \
        (void)workspace; (void)workspace_bytes;                                                     \
        int32_t st = bk::check_fp8<LAYOUT>(m, n, k, lda, ldb, c, ldc, ldd);                         \
        if (st != bk::kOk) return st;                                                               \
        if (!a || !b || !d || !bias) return bk::kInvalid;                                           \
        bk::F8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const uint8_t *)c,   \
                     ldc, d, ldd, alpha, beta, (const float *)bias};                                \
        return bk::launch_fp8<FMT, LAYOUT, bk::F8_OUT, ACTV>(p, (hipStream_t)stream);               \
    }

#define BK_FP8_BIAS_FAMILY(ENC, LAY, FMT, LAYOUT)                                                  \
    BK_FP8_BIAS_SKU(ENC, LAY, bias, FMT, LAYOUT, bk::ACT_BIAS)                                     \
    BK_FP8_BIAS_SKU(ENC, LAY, bias_relu, FMT, LAYOUT, bk::ACT_BIAS_RELU)                           \
    BK_FP8_BIAS_SKU(ENC, LAY, bias_gelu, FMT, LAYOUT, bk::ACT_BIAS_GELU)                           \
    BK_FP8_BIAS_SKU(ENC, LAY, bias_silu, FMT, LAYOUT, bk::ACT_BIAS_SILU)
