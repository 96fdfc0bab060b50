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

template <int FMT, int LAYOUT, class C>
struct F8DmaPolicy { typedef mfma2::PolicyF8<C, FMT> type; };
template <int FMT, class C>
struct F8DmaPolicy<FMT, F8_RRR, C> { typedef mfma2::PolicyF8RowB<C, FMT> type; };

// Fast path: 256x256 tiles (edge tiles included), K % 128 == 0, 16-byte rows,
// N % 4 == 0, vector stores.
template <int FMT, int LAYOUT, int EPI, int ACT, class C = F8DmaCfg>
__global__ __launch_bounds__(C::NT, C::NT == 256 ? 2 : 1) void gemm_fp8_dma_kernel(F8Args p) {
    namespace M2 = mfma2;
    typedef typename F8DmaPolicy<FMT, LAYOUT, C>::type P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * C::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * C::OPER];
    // Edge tiles (M or N not a multiple of 256): rows past M / N load as
    // zeros (past the buffer resources' byte counts; RRR B columns past N
    // read the next k-row, reaching only output columns that are not stored).
    int tm, tn;
    tile_coords(blockIdx.x, (p.M + C::TB - 1) / C::TB, (p.N + C::TB - 1) / C::TB, tm, tn);
    const int m_base = tm * C::TB, n_base = tn * C::TB;
    const bool full = m_base + C::TB <= p.M && n_base + C::TB <= p.N;
    M2::AccTile<P> acc;
    if constexpr (LAYOUT == F8_RCR) {
        M2::DmaRows<false, false> d;
        d.a = M2::make_dma_interior<C>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
        d.b = M2::make_dma_interior<C>(p.b, (uint32_t)(p.N * p.ldb), (int)p.ldb, n_base * (int)p.ldb);
        M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    } else {
        M2::DmaRowsRrr d;
        d.a = M2::make_dma_interior<C>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
        d.b = M2::make_dma_row_b<C>(p.b, (uint32_t)(p.K * p.ldb), (int)p.ldb, n_base);
        M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    }
    if constexpr (EPI == F8_BF16) {
        // bf16 rows staged per wave in LDS (free after the mainloop's last
        // barrier), written as 16-byte units: D = bf16_rne(alpha * acc).
        if (p.ldd % 8 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 8 == 0)) {
            const int wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / C::WAVES_N) * C::WM;
            const int wcol = n_base + (wave % C::WAVES_N) * C::WN;
            int8_t *scratch = (wave < C::WAVES / 2 ? stage0 : stage1) + (wave % (C::WAVES / 2)) * (C::WM * 128);
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
                min(C::WN, p.N - wcol));
            return;
        }
    }
    if constexpr (EPI == F8_F32) {
        // f32 rows staged in LDS (two halves) and written as 256-byte row
        // segments: D = alpha * acc.
        if (p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 4 == 0)) {
            const int wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / C::WAVES_N) * C::WM;
            const int wcol = n_base + (wave % C::WAVES_N) * C::WN;
            int8_t *scratch = (wave < C::WAVES / 2 ? stage0 : stage1) + (wave % (C::WAVES / 2)) * (C::WM / 2 * 256);
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
                min(C::WN, p.N - wcol));
            return;
        }
    }
    const F8Epilogue<FMT, EPI, true, ACT> epi{p};
    if constexpr (EPI == F8_OUT) {
        // fp8 bytes staged per wave, written as 16-byte row segments.
        if (p.ldd % 16 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 16 == 0)) {
            const int wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / C::WAVES_N) * C::WM;
            const int wcol = n_base + (wave % C::WAVES_N) * C::WN;
            int8_t *scratch = (wave < C::WAVES / 2 ? stage0 : stage1) + (wave % (C::WAVES / 2)) * (C::WM * C::WN);
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
                    min(C::WN, p.N - wcol));
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

// RCR last rows (1 to 16 RF of them, m0 = the first): A and B streamed
// through LDS in K stages of SB bytes, DEPTH stages in flight.  A workgroup
// of 16 waves owns 16 NB output columns; each stage holds its 16 RF A rows
// (rows past M land as zeros) then its 16 NB B rows, row r at r * SB with
// 16-byte unit u at slot u ^ (r & 15) (conflict-free fragment reads), each
// DMA instruction filling 1 KiB of it (64 consecutive units of the
// row-major stage), all issued before anything waits.  Wave w owns 128-byte
// chunk w % CH of every stage (CH = SB / 128), A row fragments
// w / CH + (16 / CH) i and all NB B fragments: one
// v_mfma_f32_16x16x128_f8f6f4 per fragment pair and stage (B rows as the
// first operand, so lane l ends with A row l % 16 and columns 4 (l / 16) ..
// + 3).  The CH chunk partials of a fragment pair are added in chunk order
// through LDS and the waves run the tiles' epilogue, one fragment pair at a
// time.  Requirements (checked by the launcher): K % SB == 0, the fast
// path's alignment and 2^31 extents, N % (16 NB) == 0; dynamic LDS of
// DEPTH * (16 RF + 16 NB) * SB bytes.
//
// RowB: B row-major [K, N] (the RRR SKUs): the stage's B region holds its SB
// k-rows of the 16 NB columns as they lie in memory (row pitch 16 NB bytes,
// whole-row DMAs, the K position moving the row by k0 * ldb); the 32 k-bytes
// of a lane's fragment come from four ds_read_b64_tr_b8 reads of 8 k-rows
// each (lane pair (2j, 2j + 1) pointing at k-row j; lane i gets 8 k of
// column i), as in PolicyF8RowB.
template <int FMT, int EPI, int ACT, int RF, int NB, int SB, int DEPTH, bool RowB = false>
__global__ __launch_bounds__(1024) void gemm_fp8_rcr_rows_staged_kernel(F8Args p, int m_first) {
    // blockIdx.y: 16 RF-row block of the pass
    const int m0 = m_first + blockIdx.y * 16 * RF;
    constexpr int WAVES = 16, CH = SB / 128;
    // With fewer (fragment, chunk) pairs than waves (RF * CH < 16) the first
    // RF * CH waves hold one each and the others only DMA.
    constexpr bool ALL = RF * CH >= WAVES;
    constexpr int FPW = ALL ? RF * CH / WAVES : 1;       // A row fragments per wave
    constexpr int FSTEP = WAVES / CH;
    constexpr int ROWS = 16 * RF + 16 * NB;              // A then B rows of a stage
    constexpr int STAGE = ROWS * SB;
    constexpr int UPR = SB / 16;                         // 16-byte units per row
    constexpr int NI = ROWS * UPR / 64;                  // 1 KiB DMA instructions per stage
    constexpr int HI = (NI + WAVES - 1) / WAVES, LO = NI / WAVES;
    static_assert((!ALL || RF * CH % WAVES == 0) && UPR >= 16 && (ROWS * UPR) % 64 == 0 && DEPTH >= 2 &&
                      DEPTH <= 4 && RF * NB * CH * 1024 <= DEPTH * STAGE,
                  "stage split");
    constexpr int F = FMT == FMT_E5M2 ? 1 : 0;
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    // RowB: a workgroup reads 16 NB-byte pieces of every k-row, so adjacent
    // column groups share 128-byte lines; workgroups go round-robin over the
    // 8 XCDs, so column groups are numbered XCD-major (consecutive groups on
    // one XCD's L2) and each line is fetched once (FETCH_SIZE 2.0x -> 1.0x of B)
    const int cgroup = RowB && gridDim.x % 8 == 0 ? (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8 : blockIdx.x;
    const int n0 = cgroup * 16 * NB;
    const v4i ra = mfma2::make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda));
    const v4i rb = mfma2::make_rsrc(p.b, (uint32_t)(RowB ? (int64_t)p.K * p.ldb : (int64_t)p.N * p.ldb));
    // DMA instruction j of a stage: units 64 j .. 64 j + 63 of the row-major
    // stage, lane L fetching unit (64 j + L) % UPR of row (64 j + L) / UPR
    auto dma_stage = [&](int st, int8_t *buf) {
        const int k0 = st * SB;
        for (int j = wave; j < NI; j += WAVES) {
            const int idx = 64 * j + lane;
            const int r = idx / UPR, slot = idx % UPR;
            const int unit = slot ^ (r & 15);
            if (r < 16 * RF) {
                mfma2::dma16(ra, (int)((int64_t)(m0 + r) * p.lda) + 16 * unit, k0, buf + j * 1024);
            } else if constexpr (RowB) {
                const int ib = idx - 16 * RF * UPR;   // unit of the B region: k-row ib / NB
                mfma2::dma16(rb, (ib / NB) * (int)p.ldb + n0 + 16 * (ib % NB),
                             __builtin_amdgcn_readfirstlane(k0 * (int)p.ldb), buf + j * 1024);
            } else {
                mfma2::dma16(rb, (int)((int64_t)(n0 + r - 16 * RF) * p.ldb) + 16 * unit, k0, buf + j * 1024);
            }
        }
    };
    const bool hi = NI % WAVES == 0 || wave < NI % WAVES;
    const int ns = p.K / SB;
    for (int st = 0; st < DEPTH && st < ns; ++st) dma_stage(st, lds + st * STAGE);
    const int c = wave % CH, f0 = wave / CH;
    const bool active = ALL || wave < RF * CH;   // wave-uniform
    v4f acc[FPW][NB];
#pragma unroll
    for (int i = 0; i < FPW; ++i)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[i][nb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // 32 bytes of K per lane: logical units 8 c + 2 g and 8 c + 2 g + 1
    const int u0 = 16 * ((8 * c + 2 * g) ^ r16), u1 = 16 * ((8 * c + 2 * g + 1) ^ r16);
    for (int st = 0; st < ns; ++st) {
        const int later = min(DEPTH - 1, ns - 1 - st);
        if (later == 0) mfma2::wait_vmcnt<0>();
        else if (later == 1) { if (hi) mfma2::wait_vmcnt<HI>(); else mfma2::wait_vmcnt<LO>(); }
        else if (later == 2) { if (hi) mfma2::wait_vmcnt<2 * HI>(); else mfma2::wait_vmcnt<2 * LO>(); }
        else { if (hi) mfma2::wait_vmcnt<3 * HI>(); else mfma2::wait_vmcnt<3 * LO>(); }
        __syncthreads();
        int8_t *buf = lds + (st % DEPTH) * STAGE;
        if (active) {
        v8i bv[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if constexpr (RowB) {
                const int kb = 128 * c + 32 * g + (r16 >> 1);
                const int8_t *q = buf + 16 * RF * SB + kb * (16 * NB) + 16 * nb + ((lane & 1) << 3);
                const mfma2::v2i_t t0 = mfma2::ds_read_tr8(q), t1 = mfma2::ds_read_tr8(q + 8 * 16 * NB);
                const mfma2::v2i_t t2 = mfma2::ds_read_tr8(q + 16 * 16 * NB), t3 = mfma2::ds_read_tr8(q + 24 * 16 * NB);
                bv[nb] = (v8i){t0[0], t0[1], t1[0], t1[1], t2[0], t2[1], t3[0], t3[1]};
            } else {
                const int8_t *brow = buf + (16 * RF + 16 * nb + r16) * SB;
                const v4i blo = *reinterpret_cast<const v4i *>(brow + u0), bhi = *reinterpret_cast<const v4i *>(brow + u1);
                bv[nb] = (v8i){blo[0], blo[1], blo[2], blo[3], bhi[0], bhi[1], bhi[2], bhi[3]};
            }
        }
#pragma unroll
        for (int i = 0; i < FPW; ++i) {
            const int8_t *arow = buf + (16 * (f0 + FSTEP * i) + r16) * SB;
            const v4i alo = *reinterpret_cast<const v4i *>(arow + u0), ahi = *reinterpret_cast<const v4i *>(arow + u1);
            const v8i av = (v8i){alo[0], alo[1], alo[2], alo[3], ahi[0], ahi[1], ahi[2], ahi[3]};
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[i][nb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bv[nb], av, acc[i][nb], F, F, 0, 0, 0, 0);
        }
        }
        __syncthreads();   // every wave is done with this buffer
        if (st + DEPTH < ns) dma_stage(st + DEPTH, buf);
    }
    // partial sums of (A fragment f, B fragment nb), chunk c: part[f][nb][c][lane]
    v4f *part = reinterpret_cast<v4f *>(lds);
    if (active) {
#pragma unroll
        for (int i = 0; i < FPW; ++i)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) part[(((f0 + FSTEP * i) * NB + nb) * CH + c) * 64 + lane] = acc[i][nb];
    }
    __syncthreads();
    const F8Epilogue<FMT, EPI, true, ACT> epi{p};
    for (int e = wave; e < RF * NB; e += WAVES) {
        const int f = e % RF, nb = e / RF;
        v4f sum = part[((f * NB + nb) * CH) * 64 + lane];
#pragma unroll
        for (int cc = 1; cc < CH; ++cc) {
            const v4f v = part[((f * NB + nb) * CH + cc) * 64 + lane];
            sum = v4f{sum[0] + v[0], sum[1] + v[1], sum[2] + v[2], sum[3] + v[3]};
        }
        epi(m0 + 16 * f + r16, n0 + 16 * nb + 4 * g, sum);   // rows past M are not stored
    }
}

// One last row (M = 1 decode steps; K % (1024 BT) == 0), no MFMA: a
// workgroup of 4 waves owns 4 output columns and wave w streams B row
// n0 + w over all of K, 16 bytes per lane of every kilobyte straight into
// registers (BT kilobytes requested before their products), beside the same
// 16 bytes of the A row (an L2 hit).  v_cvt_pk_f32_fp8 / _bf8 turn two codes
// into two f32 per instruction and f32 FMAs add the products (exact in f32,
// as in the MFMA) in a fixed per-lane order; a wave butterfly and LDS
// gather the 4 column sums and lane 0 of wave 0 runs the tiles' epilogue.
// NaN codes convert to NaN and stay NaN.
// Codes 2 HI and 2 HI + 1 of a dword (HI: the upper half) as two f32.
template <int FMT, bool HI>
__device__ __forceinline__ v2f fp8x2_to_f32(int w) {
    if constexpr (FMT == FMT_E5M2) return __builtin_amdgcn_cvt_pk_f32_bf8(w, HI);
    else return __builtin_amdgcn_cvt_pk_f32_fp8(w, HI);
}

template <int FMT, int EPI, int ACT, int BT>
__global__ __launch_bounds__(256) void gemm_fp8_rcr_row1_kernel(F8Args p, int m0) {
    __shared__ float colsum[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 4;
    const int nch = p.K >> 10;
    const int8_t *brow = p.b + (int64_t)(n0 + wave) * p.ldb + lane * 16;
    const int8_t *arow = p.a + (int64_t)m0 * p.lda + lane * 16;
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += BT) {
        v4i av[BT], bv[BT];
#pragma unroll
        for (int u = 0; u < BT; ++u) av[u] = *reinterpret_cast<const v4i *>(arow + (int64_t)(c0 + u) * 1024);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < BT; ++u)
            bv[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(brow + (int64_t)(c0 + u) * 1024));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < BT; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                const v2f a0 = fp8x2_to_f32<FMT, false>(av[u][q]), b0 = fp8x2_to_f32<FMT, false>(bv[u][q]);
                const v2f a1 = fp8x2_to_f32<FMT, true>(av[u][q]), b1 = fp8x2_to_f32<FMT, true>(bv[u][q]);
                acc0 = __builtin_fmaf(a0[0], b0[0], acc0);
                acc1 = __builtin_fmaf(a0[1], b0[1], acc1);
                acc0 = __builtin_fmaf(a1[0], b1[0], acc0);
                acc1 = __builtin_fmaf(a1[1], b1[1], acc1);
            }
    }
    float acc = acc0 + acc1;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) colsum[wave] = acc;
    __syncthreads();
    if (threadIdx.x != 0) return;
    const F8Epilogue<FMT, EPI, true, ACT> epi{p};
    epi(m0, n0, v4f{colsum[0], colsum[1], colsum[2], colsum[3]});
}

// Stage shapes of the FP8 last-rows kernel (first match wins), by the
// column fragments per workgroup (mfma2::last_rows_col_frags).  N = 14336,
// K = 4096 over 8 rotated weight sets (HIP events), 64 columns per
// workgroup: up to 64 rows with 4 fragments and 512-byte stages, M = 1 / 16
// / 32 / 64 in 14.2 / 14.3 / 14.6 / 15.6 us (48 us on 256-row tiles; 16
// columns with 1 / 2 / 4 fragments: 16.1 / 17.5 / 20.7 / 23.4); 65-128 rows
// with 8 fragments and 256-byte stages, M = 65 / 100 / 128 in 17.8 / 18.5 /
// 20.0 us (16 columns: 35.0 / 36.8 / 38.0; 32: 22.9 / 24.2 / 26.1; 128
// columns 24.2-25.9).  16 columns (N below 6144): 1 fragment with 2 KiB
// stages, 2 with 1 KiB stages three deep, 4 and 8 with 512-byte stages.
template <int FMT, int EPI, int ACT>
bool launch_fp8_rows(const F8Args &p, int m0, int rem, hipStream_t stream) {
    // one row: the FMA row kernel (K = 4096 over rotated weights, graph
    // replay: N = 14336 13.4 -> 10.4 us, N = 4096 5.2 -> 4.8 us against the
    // staged kernel)
    if (rem == 1 && p.K % 1024 == 0) {
        if (p.K % 2048 == 0)
            hipLaunchKernelGGL((gemm_fp8_rcr_row1_kernel<FMT, EPI, ACT, 2>), dim3(p.N / 4), dim3(256), 0, stream, p, m0);
        else
            hipLaunchKernelGGL((gemm_fp8_rcr_row1_kernel<FMT, EPI, ACT, 1>), dim3(p.N / 4), dim3(256), 0, stream, p, m0);
        return true;
    }
    if (rem > 32 && mfma2::last_rows_col_frags(p.N) == 1) {
        // 33-128 rows below N = 6144 as row blocks (mfma2::last_rows_blocks);
        // 32-row blocks need 1 KiB stages here (a wave's 128-byte chunks
        // must cover the 16 waves), which fit LDS up to 32 columns.  K =
        // 4096, graph replay, rotated weights, M = 48 / 100 / 128: N = 4096
        // 7.6 / 10.4 / 10.7 -> 6.8 / 8.1 / 8.1 us; N = 2048 7.0 / 9.5 / 9.6
        // -> 5.3 / 6.0 / 6.2 us; N = 3072 7.1 / 9.7 / 9.9 -> 6.0 / 8.0 / 8.0
        int rf, blk, nbb;
        mfma2::last_rows_blocks(rem, p.N, rf, blk, nbb);
#define BK_F8RB(RF, NB, SB, DEPTH)                                                                        \
        if (rf == (RF) && nbb == (NB) && p.K % (SB) == 0) {                                                  \
            hipLaunchKernelGGL((gemm_fp8_rcr_rows_staged_kernel<FMT, EPI, ACT, RF, NB, SB, DEPTH>),           \
                               dim3(p.N / (16 * (NB)), blk), dim3(1024), (size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), \
                               stream, p, m0);                                                               \
            return true;                                                                                     \
        }
        BK_F8RB(4, 1, 512, 2) BK_F8RB(4, 2, 512, 2) BK_F8RB(4, 4, 512, 2)
        BK_F8RB(2, 1, 1024, 3) BK_F8RB(2, 2, 1024, 2)
#undef BK_F8RB
    }
    const int nb = mfma2::last_rows_col_frags(p.N);
#define BK_F8ROWS(RF, NB, SB, DEPTH)                                                                     \
    if (rem <= 16 * (RF) && nb == (NB) && p.K % (SB) == 0) {                                              \
        hipLaunchKernelGGL((gemm_fp8_rcr_rows_staged_kernel<FMT, EPI, ACT, RF, NB, SB, DEPTH>),           \
                           dim3(p.N / (16 * (NB))), dim3(1024), (size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), \
                           stream, p, m0);                                                               \
        return true;                                                                                     \
    }
    // up to 16 / 32 rows at 32 or 64 columns: 1 / 2 fragments, 4 / 8 waves
    // with MFMA work (padding A rows cost DMA and LDS time: N = 14336, M = 2
    // / 8 / 16 / 32 14.7 / 14.0 / 13.3 / 13.6 -> 13.4 / 12.8 / 12.3 / 12.9 us
    // against 4 fragments; N = 8192, M = 2-16 8.9 -> 8.35 us)
    BK_F8ROWS(1, 4, 512, 2)
    BK_F8ROWS(2, 4, 512, 2)
    BK_F8ROWS(1, 2, 512, 2)
    BK_F8ROWS(2, 2, 512, 2)
    BK_F8ROWS(4, 4, 512, 2)
    BK_F8ROWS(8, 4, 256, 2)
    BK_F8ROWS(4, 2, 512, 2)
    BK_F8ROWS(8, 2, 512, 2)
    BK_F8ROWS(1, 1, 2048, 2)
    BK_F8ROWS(2, 1, 1024, 3)
    BK_F8ROWS(4, 1, 512, 2)
    BK_F8ROWS(8, 1, 512, 2)
#undef BK_F8ROWS
    return false;
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
    if (fast && LAYOUT == F8_RRR && p.K % 512 == 0 && (int64_t)p.K * p.ldb + mfma2::BN < (1ll << 31)) {
        // RRR last rows: the staged kernel reading row-major B, column groups
        // by the last-rows rule (XCD-major in the kernel)
        const int rem = mfma2::last_rows_pass(p.M, p.N, 128);
        if (rem == 0 && p.M > 128 && p.M <= 512 && p.N % 16 == 0) {
            // a small grid: every row as row blocks of the same kernel (64-row
            // blocks, else 128-row) while they fit one round of workgroups.
            // K = 4096, M = 129 / 256 / 512 against 256x256 RRR tiles: N =
            // 4096 38.9 / 40.3 / 40.2 -> 17.4 / 17.4 / 27.1 us, N = 2048
            // 38.7 / 40.8 / 40.7 -> 10.7 / 11.3 / 17.4 us
            const int b4 = (p.M + 63) / 64, n4 = mfma2::last_rows_col_frags(p.N, b4);
            const int b8 = (p.M + 127) / 128, n8 = mfma2::last_rows_col_frags(p.N, b8);
            const bool use4 = b4 * (p.N / (16 * n4)) <= 256;
            const int blk = use4 ? b4 : b8, nbb = use4 ? n4 : n8;
            if (blk * (p.N / (16 * nbb)) <= 256) {
#define BK_F8RRRW(RF, NB, SB)                                                                             \
                if ((use4 ? 4 : 8) == (RF) && nbb == (NB)) {                                                 \
                    hipLaunchKernelGGL((gemm_fp8_rcr_rows_staged_kernel<FMT, EPI, ACT, RF, NB, SB, 2, true>), \
                                       dim3(p.N / (16 * (NB)), blk), dim3(1024),                             \
                                       (size_t)2 * (16 * (RF) + 16 * (NB)) * (SB), stream, p, 0);            \
                    return launch_status();                                                                  \
                }
                BK_F8RRRW(4, 1, 512) BK_F8RRRW(4, 2, 512) BK_F8RRRW(4, 4, 512)
                BK_F8RRRW(8, 1, 512) BK_F8RRRW(8, 2, 512) BK_F8RRRW(8, 4, 256)
#undef BK_F8RRRW
            }
        }
        if (rem != 0) {
            F8Args pm = p;
            pm.M = p.M - rem;
            const int tiles = (pm.M / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
            if (tiles > 0)
                hipLaunchKernelGGL((gemm_fp8_dma_kernel<FMT, LAYOUT, EPI, ACT>), dim3(tiles), dim3(F8DmaCfg::NT),
                                   0, stream, pm);
            if (rem > 32 && mfma2::last_rows_col_frags(p.N) == 1) {
                // row blocks as the RCR pass (K = 4096, M = 100: N = 4096
                // 13.8 -> 11.7 us, N = 2048 12.8 -> 9.8 us)
                int rf, blk, nbb;
                mfma2::last_rows_blocks(rem, p.N, rf, blk, nbb);
#define BK_F8RRRB(RF, NB, SB, DEPTH)                                                                      \
                if (rf == (RF) && nbb == (NB) && p.K % (SB) == 0) {                                          \
                    hipLaunchKernelGGL((gemm_fp8_rcr_rows_staged_kernel<FMT, EPI, ACT, RF, NB, SB, DEPTH, true>), \
                                       dim3(p.N / (16 * (NB)), blk), dim3(1024),                             \
                                       (size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), stream, p, pm.M);   \
                    return launch_status();                                                                  \
                }
                BK_F8RRRB(4, 1, 512, 2) BK_F8RRRB(4, 2, 512, 2) BK_F8RRRB(4, 4, 512, 2)
                BK_F8RRRB(2, 1, 1024, 3) BK_F8RRRB(2, 2, 1024, 2)
#undef BK_F8RRRB
            }
            const int nb = mfma2::last_rows_col_frags(p.N);
#define BK_F8RRRROWS(RF, NB, SB, DEPTH)                                                                    \
            if (rem <= 16 * (RF) && nb == (NB)) {                                                         \
                hipLaunchKernelGGL((gemm_fp8_rcr_rows_staged_kernel<FMT, EPI, ACT, RF, NB, SB, DEPTH, true>), \
                                   dim3(p.N / (16 * (NB))), dim3(1024),                                  \
                                   (size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), stream, p, pm.M);    \
                return launch_status();                                                                   \
            }
            // up to 16 / 32 rows: 1 / 2 fragments with 4 / 8 waves
            // multiplying (K = 4096: M = 1-16 N = 4096 9.1 -> 8.8 us, N =
            // 14336 18.4 -> 13.5 us; M = 17-32 N = 8192 12.6 -> 11.9 us, N =
            // 14336 18.3 -> 14.5 us)
            BK_F8RRRROWS(1, 1, 512, 3)
            BK_F8RRRROWS(1, 2, 512, 3)
            BK_F8RRRROWS(1, 4, 512, 3)
            BK_F8RRRROWS(2, 2, 512, 2)
            BK_F8RRRROWS(2, 4, 512, 2)
            BK_F8RRRROWS(4, 4, 512, 2)
            BK_F8RRRROWS(8, 4, 256, 2)
            BK_F8RRRROWS(4, 2, 512, 2)
            BK_F8RRRROWS(8, 2, 512, 2)
            BK_F8RRRROWS(2, 1, 1024, 3)
            BK_F8RRRROWS(4, 1, 512, 2)
            BK_F8RRRROWS(8, 1, 512, 2)
#undef BK_F8RRRROWS
        }
    }
    if (fast && LAYOUT == F8_RCR && p.M > 128 && p.M <= 512 && p.K % 512 == 0 && p.N % 16 == 0 &&
        mfma2::last_rows_pass(p.M, p.N, 128) == 0) {
        // small problems whose 128-row blocks of the last-rows kernel fit one
        // round of workgroups: all rows that way instead of tiles.  K = 4096,
        // M = 129 / 256 / 512: N = 4096 12.6 / 13.2 / 18.6 us against 23.9 /
        // 24.2 / 24.3 on 128x128 tiles; N = 8192, M = 129 / 256: 17.5 / 18.6
        // against 28.2 / 28.6
        // 64-row blocks first while they fit one round (K = 4096, M = 129 /
        // 256: N = 4096 12.3 / 12.8 -> 11.2 / 11.7 us, N = 2048 9.6 / 10.1
        // -> 7.9 / 8.1 us; N = 8192 level), else 128-row blocks
        const int b4 = (p.M + 63) / 64;
        const int n4 = mfma2::last_rows_col_frags(p.N, b4);
        if (b4 * (p.N / (16 * n4)) <= 256) {
#define BK_F8BLK4(NB)                                                                                     \
            if (n4 == (NB)) {                                                                             \
                hipLaunchKernelGGL((gemm_fp8_rcr_rows_staged_kernel<FMT, EPI, ACT, 4, NB, 512, 2>),        \
                                   dim3(p.N / (16 * (NB)), b4), dim3(1024), (size_t)2 * (64 + 16 * (NB)) * 512, \
                                   stream, p, 0);                                                         \
                return launch_status();                                                                   \
            }
            BK_F8BLK4(1) BK_F8BLK4(2) BK_F8BLK4(4)
#undef BK_F8BLK4
        }
        const int blocks = (p.M + 127) / 128;
        const int nb = mfma2::last_rows_col_frags(p.N, blocks);
        if (blocks * (p.N / (16 * nb)) <= 256) {
#define BK_F8BLOCKS(NB, SB)                                                                              \
            if (nb == (NB)) {                                                                            \
                hipLaunchKernelGGL((gemm_fp8_rcr_rows_staged_kernel<FMT, EPI, ACT, 8, NB, SB, 2>),        \
                                   dim3(p.N / (16 * (NB)), blocks), dim3(1024),                          \
                                   (size_t)2 * (128 + 16 * (NB)) * (SB), stream, p, 0);                  \
                return launch_status();                                                                  \
            }
            BK_F8BLOCKS(1, 512)
            BK_F8BLOCKS(2, 512)
            BK_F8BLOCKS(4, 256)
#undef BK_F8BLOCKS
        }
    }
    if (fast && LAYOUT == F8_RCR) {
        // the last rows as their own pass when a row of tiles would start
        // another round (decode-sized M: all of it)
        const int rem = mfma2::last_rows_pass(p.M, p.N, 128);
        if (rem != 0 && p.K % 512 == 0) {
            F8Args pm = p;
            pm.M = p.M - rem;
            const int tiles = (pm.M / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
            if (tiles > 0)
                hipLaunchKernelGGL((gemm_fp8_dma_kernel<FMT, LAYOUT, EPI, ACT>), dim3(tiles), dim3(F8DmaCfg::NT),
                                   0, stream, pm);
            if (launch_fp8_rows<FMT, EPI, ACT>(p, pm.M, rem, stream)) return launch_status();
            // K % 512 == 0 always finds a stage shape
        }
    }
    if (fast) {
        const int tiles = (int)(pad_m / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
        if (LAYOUT == F8_RCR && tiles <= 128) {
            // at most half a round of 256x256 tiles: 128x128 tiles of 4 waves
            // (two workgroups per CU), as the int8 kernel
            typedef mfma2::Cfg<2, 2, 128> SmallCfg;
            const int tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128);
            hipLaunchKernelGGL((gemm_fp8_dma_kernel<FMT, F8_RCR, EPI, ACT, SmallCfg>), dim3(tiles128),
                               dim3(SmallCfg::NT), 0, stream, p);
            return launch_status();
        }
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
